"""Parity of the generated HIP executors with the CPU oracle.

Tolerances.  Where the floating-point evaluation order is the sequential
loop's (one lane per task, ILU0's per-entry updates, the mailbox protocol)
the results must be bit-identical (device code is compiled with
-ffp-contract=off).  Where the order differs -- atomic accumulation in CSC
SpTRSV, lane-strided partial sums with a butterfly reduction in CSR SpTRSV --
the check is element-wise, as the reference's own is
(compiler/e2e_tests/test_sptrsv_e2e.py:64-69, rtol 1e-10 / atol 1e-12), at
the tighter north-star bound:

    |x_i - ref_i| <= 1e-12 * |ref_i| + 1e-15 * max|ref|     for every i

(the absolute floor, 1e-15 of the largest entry, keeps entries that cancel
to almost nothing from demanding more digits than the sums that form them
carry).  ``elementwise_error`` returns max_i |x_i - ref_i| / (|ref_i| +
1e-3 max|ref|), which is at most 1e-12 exactly when the bound holds.
"""

import ast
import inspect

import numpy as np
import pytest

from lcd_amd import workloads
from lcd_amd.demo import gauss_seidel, spilu0, sptrsv

pytestmark = pytest.mark.gpu
TOLERANCE = 1e-12
ABSOLUTE_FLOOR = 1e-15


def elementwise_error(result, expected):
    result, expected = np.asarray(result), np.asarray(expected)
    scale = float(np.max(np.abs(expected))) or 1.0
    floor = scale * ABSOLUTE_FLOOR / TOLERANCE
    return float(np.max(np.abs(result - expected)
                        / (np.abs(expected) + floor)))


relative_error = elementwise_error


def solve_and_check(solver, work, expected, exact=False):
    result = solver(work.indptr, work.indices, work.data, work.rhs, work.n)
    assert result.shape == expected.shape
    if exact:
        np.testing.assert_array_equal(result, expected)
    else:
        assert elementwise_error(result, expected) <= TOLERANCE
    return result


CSC_VARIANTS = [
    dict(execution_mode="wavefront", threads_per_block=128, task_lanes=4),
    dict(execution_mode="wavefront", threads_per_block=128, n_warp=1),
    dict(execution_mode="wavefront", threads_per_block=256, task_lanes=8,
         thread_unroll=2),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=8,
         dependence_protocol="push"),
    dict(execution_mode="sync_free", threads_per_block=128, n_warp=1,
         dependence_protocol="push"),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4,
         dependence_protocol="counter"),
    dict(execution_mode="wavefront", threads_per_block=128, n_warp=2),
    dict(execution_mode="sync_free", threads_per_block=128, n_warp=2),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=4,
         dependence_protocol="mailbox"),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=2,
         dependence_protocol="mailbox", thread_unroll=2),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=4,
         dependence_protocol="mailbox", gather_messages=False),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=8,
         dependence_protocol="mailbox", gather_messages=False,
         thread_unroll=2),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4,
         dependence_protocol="mailbox", tile_rows=None),
    dict(execution_mode="sync_free", threads_per_block=128, n_warp=1,
         dependence_protocol="mailbox"),
    # gathered operands staged per launch instead of read through records
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4,
         dependence_protocol="mailbox", tile_rows=None, task_records=False),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4,
         dependence_protocol="mailbox", tile_rows=256, task_records=False),
    dict(),   # scheduler decides
]


@pytest.mark.parametrize("options", CSC_VARIANTS, ids=lambda o: "-".join(
    f"{k}={v}" for k, v in o.items()) or "auto")
def test_sptrsv_csc_variants(oracle, options):
    print("csc", options, flush=True)
    solver = sptrsv.compile_sptrsv_csc(**options)
    # the mailbox protocol adds the incoming products in the order of the
    # sequential loop: bit-identical results, not just 1e-12
    defaulted = (options.get("execution_mode") == "sync_free"
                 and "dependence_protocol" not in options
                 and options.get("n_warp", 1) == 1)
    exact = options.get("dependence_protocol") == "mailbox" or defaulted
    for name, overrides in (("c1", {}), ("c2", dict(nx=20, ny=18, nz=16)),
                            ("c5", dict(n=6000))):
        work = workloads.configuration(name, **overrides)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(solver, work, expected, exact=exact)
    if exact:
        assert solver.current_schedule.dependence_protocol == "mailbox"
        slots = "_lcd_mailbox" in solver.hip_kernel_source
        # message slots only when the (default) gathered form is off
        assert slots == (options.get("gather_messages") is False)
        assert ("_lcd_in_src" in solver.hip_kernel_source) != slots
    schedule = solver.current_schedule
    if "execution_mode" in options:
        assert schedule.execution_mode == options["execution_mode"]
    if options.get("dependence_protocol") == "push":
        assert schedule.dependence_protocol == "push"
        assert "_lcd_mailbox" not in solver.hip_kernel_source


@pytest.mark.parametrize("lanes", [1, 4, 8, 64])
def test_level_launches_gather_their_products(oracle, lanes):
    """Level launches of the CSC solve: a task adds the products of its
    incoming entries itself, in the order of the sequential loop, instead of
    its producers pushing them with atomics -- no atomics, the same bits in
    every run and as the sequential loop; in-degrees below, at and above the
    lanes of a task (several chunks)."""
    print("level gather", lanes, flush=True)
    gathered = sptrsv.compile_sptrsv_csc(
        execution_mode="wavefront", threads_per_block=128, task_lanes=lanes,
        thread_unroll=1)
    pushed = sptrsv.compile_sptrsv_csc(
        execution_mode="wavefront", threads_per_block=128, task_lanes=lanes,
        thread_unroll=1, level_gather=False)
    assert gathered.hip_lowering.dependence_protocol == "mailbox"
    assert pushed.hip_lowering.dependence_protocol == "counter"
    assert "lcd_atomic" not in gathered.hip_kernel_source
    assert "_lcd_in_src[" in gathered.hip_kernel_source
    assert "lcd_atomic_add" in pushed.hip_kernel_source
    for name, overrides in (("c1", {}), ("c2", dict(nx=20, ny=18, nz=16)),
                            ("c5", dict(n=6000))):
        work = workloads.configuration(name, **overrides)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        for _ in range(2):
            solve_and_check(gathered, work, expected, exact=True)
        solve_and_check(pushed, work, expected)
    # the operands of a launch lie in level order (staged copies): other
    # matrix values and another right-hand side through the same plan
    assert gathered.hip_lowering.level_records
    assert gathered.hip_lowering.task_record_lanes == max(lanes, 4 if lanes == 1
                                                          else lanes)
    work = workloads.configuration("c2", nx=20, ny=18, nz=16)
    rng = np.random.default_rng(lanes)
    for _ in range(2):
        values = work.data * rng.uniform(0.5, 1.5, len(work.data))
        rhs = rng.standard_normal(work.n)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, values, rhs,
                                     work.n)
        np.testing.assert_array_equal(
            gathered(work.indptr, work.indices, values, rhs, work.n), expected)
    # a power-law factor: hundreds of incoming entries for some rows
    lower, diagonal, rhs = random_lower_factor(3000, 7)
    import scipy.sparse as sp
    matrix = sp.csc_matrix(lower + sp.diags(diagonal))
    matrix.sort_indices()
    indptr, indices = (matrix.indptr.astype(np.int32),
                       matrix.indices.astype(np.int32))
    expected = oracle.sptrsv_csc(indptr, indices, matrix.data, rhs, 3000)
    np.testing.assert_array_equal(
        gathered(indptr, indices, matrix.data, rhs, 3000), expected)
    # chain tasks (band_width > 1) keep their counters
    banded = sptrsv.compile_sptrsv_csc(
        execution_mode="wavefront", threads_per_block=128, task_lanes=lanes,
        thread_unroll=1, band_width=4)
    assert banded.hip_lowering.dependence_protocol == "counter"


@pytest.mark.parametrize("tile_rows,lanes,tpb", [(64, 4, 64), (500, 8, 128),
                                                 (4096, 4, 256), (8192, 16, 512),
                                                 (256, 2, 128)])
def test_tiled_executor(oracle, tile_rows, lanes, tpb):
    """Workgroup-resident tiles: hand-offs inside a tile go through LDS,
    across tiles through memory; CSR pull and the gathered CSC mailbox."""
    print("tiles", tile_rows, lanes, tpb, flush=True)
    csr = sptrsv.compile_sptrsv_csr(
        execution_mode="sync_free", threads_per_block=tpb, task_lanes=lanes,
        thread_unroll=1, dependence_protocol="pull", tile_rows=tile_rows)
    csc = sptrsv.compile_sptrsv_csc(
        execution_mode="sync_free", threads_per_block=tpb, task_lanes=lanes,
        thread_unroll=1, dependence_protocol="mailbox", gather_messages=True,
        tile_rows=tile_rows, tile_box=None)      # tiles of consecutive ids
    assert csr.hip_lowering.tile_rows == tile_rows
    assert csc.hip_lowering.tile_rows == tile_rows
    assert "lcd_tile_ld(x, _lcd_tile" in csr.hip_kernel_source
    assert "lcd_tile_st(x, _lcd_tile" in csc.hip_kernel_source
    # the first `lanes` incoming edges of a task come from its record
    assert csc.hip_lowering.task_record_lanes == lanes
    assert "_lcd_rec_src[" in csc.hip_kernel_source
    assert csc.hip_lowering.stage_kernel_name is None
    for name, overrides in (("c1", {}), ("c2", dict(nx=20, ny=18, nz=16)),
                            ("c5", dict(n=6000))):
        work = workloads.configuration(name, **overrides)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        # the gathered mailbox adds in the order of the sequential loop
        solve_and_check(csc, work, expected, exact=True)
        # in-degrees: 2 (c1), 3 (c2), 8 (c5); the executor variant without
        # the code for a second chunk runs exactly when they fit the record
        in_degree = {"c1": 2, "c2": 3, "c5": 8}[name]
        plan = csc.schedule_plan(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
        assert plan.single_chunk == (in_degree <= lanes)
        assert ("_lcd_in_src[_mb_next + _lane]" in csc.hip_kernel_source) == (
            in_degree > lanes)
    work = workloads.configuration("c3", n=20000)
    expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solve_and_check(csr, work, expected)
    # a loop the tiles do not apply to keeps the flat queue
    pushed = sptrsv.compile_sptrsv_csc(
        execution_mode="sync_free", threads_per_block=128, task_lanes=4,
        thread_unroll=1, dependence_protocol="push", tile_rows=tile_rows)
    assert pushed.hip_lowering.tile_rows is None


@pytest.mark.parametrize("box,lanes,tpb", [((8, 4, 4), 4, 128),
                                           ((20, 3, 2), 4, 64),
                                           ((5, 5, 5), 8, 256),    # ragged
                                           ("auto", 4, 256)])
def test_box_tiles(oracle, box, lanes, tpb):
    """Tiles over boxes of the grid: the LDS copy and the value-as-flag
    buffer are addressed by the place of a task in the queue, the result is
    that of the sequential loop bit for bit; structures that are no grid, or
    whose tasks have more incoming edges than lanes, keep tiles of
    consecutive ids."""
    print("box tiles", box, lanes, tpb, flush=True)
    csc = sptrsv.compile_sptrsv_csc(
        execution_mode="sync_free", threads_per_block=tpb, task_lanes=lanes,
        thread_unroll=1, dependence_protocol="mailbox", tile_rows=256,
        tile_box=box)
    for name, overrides, boxed in (
            ("c2", dict(nx=20, ny=18, nz=16), True),
            # two axes: a box chosen by the scheduler would be consecutive
            # lines, which tiles of consecutive ids are already
            ("c1", {}, box != "auto"),
            ("c5", dict(n=6000), False)):          # a band, no grid
        work = workloads.configuration(name, **overrides)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        for _ in range(2):      # the second call reuses the plan's buffers
            solve_and_check(csc, work, expected, exact=True)
        plan = csc.schedule_plan(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
        assert (plan.tile_boxes is not None) == boxed, name
        assert csc.hip_lowering.tile_by_position == boxed
        assert ("_lcd_xq[" in csc.hip_kernel_source) == boxed
        if boxed and name == "c2":
            assert plan.tile_boxes[0] == (20, 18, 16)
            if box != "auto":
                assert plan.tile_boxes[1] == box
                assert plan.tile_rows == box[0] * box[1] * box[2]
            else:
                assert np.prod(plan.tile_boxes[1]) <= 256
    with pytest.raises(ValueError):
        sptrsv.compile_sptrsv_csc(tile_box=(4, 4))
    # a grid given by the caller that the structure does not have: the
    # order is not topological, the plan falls back to consecutive ids
    wrong = sptrsv.compile_sptrsv_csc(
        execution_mode="sync_free", threads_per_block=128, task_lanes=4,
        thread_unroll=1, dependence_protocol="mailbox", tile_rows=256,
        tile_box=(2, 2, 1), tile_grid=(4, 2, 720))
    work = workloads.configuration("c2", nx=20, ny=18, nz=16)
    expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solve_and_check(wrong, work, expected, exact=True)
    assert wrong.schedule_plan(work.indptr, work.indices, work.data, work.rhs,
                               work.n).tile_boxes is None


def test_box_tiles_divide_again_outside_the_prepared_range(oracle):
    """The box tiles divide over a reciprocal prepared a round ahead; a
    divisor or a quotient outside the range that serves (tiny, huge,
    denormal, zero, not finite) is divided again in full, per lane: the
    sequential loop's bits, and the same bits without the preparation."""
    work = workloads.configuration("c2", nx=20, ny=18, nz=16)
    options = dict(execution_mode="sync_free", threads_per_block=128,
                   task_lanes=4, thread_unroll=1,
                   dependence_protocol="mailbox", tile_rows=256,
                   tile_box=(20, 3, 2))
    prepared = sptrsv.compile_sptrsv_csc(**options)
    plain = sptrsv.compile_sptrsv_csc(prepared_division=False, **options)
    values = work.data.copy()
    rhs = work.rhs.copy()
    diagonal = work.indptr[:-1]
    values[diagonal[50]] = 1e-200
    values[diagonal[51]] = 1e250
    values[diagonal[200]] = 5e-324
    values[diagonal[777]] = -3e-120
    values[diagonal[1500]] = 2.0 ** 100
    rhs[300], rhs[301], rhs[4000] = 1e-305, 0.0, -0.0
    rhs[2500] = np.inf
    with np.errstate(all="ignore"):
        expected = oracle.sptrsv_csc(work.indptr, work.indices, values, rhs,
                                     work.n)
    for solver in (prepared, plain):
        result = solver(work.indptr, work.indices, values, rhs, work.n)
        np.testing.assert_array_equal(result, expected)
        valid = ~np.isnan(expected)
        np.testing.assert_array_equal(np.signbit(result[valid]),
                                      np.signbit(expected[valid]))
    assert "LCD_PREPARED_DIVISION 1" in prepared.hip_lowering.source
    assert "LCD_PREPARED_DIVISION 1" not in plain.hip_lowering.source


def random_lower_factor(n, seed):
    """Lower-triangular factor with a skewed row-length mix: empty rows,
    short rows and a few rows with up to 300 entries (more incoming edges
    than any lane count), unit-scale values, dominant diagonal."""
    import scipy.sparse as sp
    rng = np.random.default_rng(seed)
    rows, cols = [], []
    for i in range(1, n):
        kind = rng.random()
        count = (0 if kind < 0.1 else int(rng.integers(1, 6)) if kind < 0.9
                 else int(rng.integers(20, 300)))
        count = min(count, i)
        # mostly nearby columns, some far ones
        near = max(0, i - 40)
        picks = np.unique(np.concatenate([
            rng.integers(near, i, size=count),
            rng.integers(0, i, size=max(count // 4, 0))]))
        rows += [i] * len(picks)
        cols += picks.tolist()
    values = rng.uniform(-1.0, 1.0, len(rows))
    lower = sp.csr_matrix((values, (rows, cols)), shape=(n, n))
    diagonal = 1.0 + np.asarray(abs(lower).sum(axis=1)).ravel()
    return lower, diagonal, rng.standard_normal(n)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_factors_through_every_persistent_executor(oracle, seed):
    """Random structure (not a stencil): empty rows, in-degrees beyond the
    record size, edges near and far -- CSC and CSR, flat and tiled."""
    import scipy.sparse as sp
    n = 3000 + 517 * seed
    print("random factor", seed, n, flush=True)
    lower, diagonal, rhs = random_lower_factor(n, seed)
    # CSC with the diagonal first, CSR with the diagonal last
    csc = sp.csc_matrix(lower + sp.diags(diagonal))
    csc.sort_indices()
    csr = sp.csr_matrix(lower + sp.diags(diagonal))
    csr.sort_indices()
    by_column = tuple(a.astype(np.int32) for a in (csc.indptr, csc.indices))
    by_row = tuple(a.astype(np.int32) for a in (csr.indptr, csr.indices))
    expected_csc = oracle.sptrsv_csc(*by_column, csc.data, rhs, n)
    expected_csr = oracle.sptrsv_csr(*by_row, csr.data, rhs, n)
    assert relative_error(expected_csc, expected_csr) <= 1e-10
    for options in (dict(task_lanes=4, tile_rows=None),
                    dict(task_lanes=8, tile_rows=256),
                    dict(task_lanes=64, tile_rows=None),
                    dict(task_lanes=4, tile_rows=None, task_records=False),
                    dict(task_lanes=16, tile_rows=None, gather_messages=False)):
        print("  csc", options, flush=True)
        solver = sptrsv.compile_sptrsv_csc(
            execution_mode="sync_free", threads_per_block=128,
            thread_unroll=1, dependence_protocol="mailbox", **options)
        result = solver(*by_column, csc.data, rhs, n)
        # incoming products are added in the sequential order: bit-identical
        np.testing.assert_array_equal(result, expected_csc)
        if options.get("task_records", True) and options.get(
                "gather_messages", True):
            plan = solver.schedule_plan(*by_column, csc.data, rhs, n)
            assert plan.dag.record_overflow > 0 or options["task_lanes"] == 64
            assert plan.single_chunk == (plan.dag.record_overflow == 0)
    for options in (dict(task_lanes=8, tile_rows=None),
                    dict(task_lanes=32, tile_rows=512),
                    dict(task_lanes=16, tile_rows=None, value_flags=False)):
        print("  csr", options, flush=True)
        solver = sptrsv.compile_sptrsv_csr(
            execution_mode="sync_free", threads_per_block=128,
            thread_unroll=1, dependence_protocol="pull", **options)
        result = solver(*by_row, csr.data, rhs, n)
        assert relative_error(result, expected_csr) <= TOLERANCE


CSR_VARIANTS = [
    dict(execution_mode="wavefront", threads_per_block=128, task_lanes=8),
    dict(execution_mode="wavefront", threads_per_block=128, n_warp=1,
         thread_unroll=4),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=8,
         dependence_protocol="pull"),
    dict(execution_mode="sync_free", threads_per_block=128, n_warp=1,
         dependence_protocol="pull"),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=16,
         dependence_protocol="counter"),
    dict(execution_mode="wavefront", threads_per_block=256, n_warp=4),
    dict(),
]


@pytest.mark.parametrize("options", CSR_VARIANTS, ids=lambda o: "-".join(
    f"{k}={v}" for k, v in o.items()) or "auto")
def test_sptrsv_csr_variants(oracle, options):
    print("csr", options, flush=True)
    solver = sptrsv.compile_sptrsv_csr(**options)
    work = workloads.configuration("c3", n=20000)
    expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solve_and_check(solver, work, expected)
    if options.get("dependence_protocol"):
        assert (solver.current_schedule.dependence_protocol
                == options["dependence_protocol"])


def test_sptrsv_csr_lane_per_task_is_bit_exact(oracle):
    """No thread map: each task runs the sequential row loop on one lane."""
    work = workloads.configuration("c3", n=20000)
    expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solve_and_check(sptrsv.simple_sptrsv_csr, work, expected, exact=True)
    from lcd_amd import parallel
    sync_free = parallel(loop="i", function_props=sptrsv.FUNCTION_PROPS_CSR,
                         execution_mode="sync_free")(sptrsv.sptrsv_csr_loop)
    solve_and_check(sync_free, work, expected, exact=True)


def test_sptrsv_matches_scipy_and_manufactured_solution(oracle):
    """The reference's own e2e oracle (test_sptrsv_e2e.py:58-69) and its
    demo's manufactured solution (demo/sptrsv.py:51-52)."""
    from scipy.sparse import csc_matrix
    from scipy.sparse.linalg import spsolve_triangular
    work = workloads.configuration("c2", nx=16, ny=16, nz=16)
    matrix = csc_matrix((work.data, work.indices, work.indptr),
                        shape=(work.n, work.n))
    expected = np.linspace(1.0, 2.0, work.n)
    rhs = np.asarray(matrix @ expected).ravel()
    result = sptrsv.simple_sptrsv_csc(work.indptr, work.indices, work.data,
                                      rhs, work.n)
    np.testing.assert_allclose(result, expected, rtol=1e-10, atol=1e-12)
    reference = spsolve_triangular(matrix.tocsr(), rhs, lower=True)
    np.testing.assert_allclose(result, reference, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("tile_rows,tpb,waves_per_cu",
                         [(128, 384, None), (64, 64, 1), (256, 192, 2)])
def test_more_tiles_than_workgroups(oracle, tile_rows, tpb, waves_per_cu):
    """More tiles than the persistent grid has workgroups: the tiles are
    claimed from the task counter, so the run does not depend on every
    workgroup of the grid being resident at the same time (six wavefronts
    per workgroup do not spread evenly over four SIMDs, and the occupancy
    query then promises more workgroups than the CUs hold). The first case
    has 1536 tiles of six wavefronts each, more than any grid of them; the
    others cap the grid far below their tile counts."""
    work = workloads.configuration("c2", nx=64, ny=64, nz=48)
    expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    csc = sptrsv.compile_sptrsv_csc(
        execution_mode="sync_free", threads_per_block=tpb, task_lanes=4,
        dependence_protocol="mailbox", tile_rows=tile_rows,
        resident_waves_per_cu=waves_per_cu)
    solve_and_check(csc, work, expected, exact=True)
    assert "_lcd_claim" in csc.hip_kernel_source
    matrix_rows = workloads.configuration("c3", n=150000)
    csr = sptrsv.compile_sptrsv_csr(
        execution_mode="sync_free", threads_per_block=tpb, task_lanes=8,
        dependence_protocol="pull", tile_rows=tile_rows,
        resident_waves_per_cu=waves_per_cu)
    expected = oracle.sptrsv_csr(matrix_rows.indptr, matrix_rows.indices,
                                 matrix_rows.data, matrix_rows.rhs,
                                 matrix_rows.n)
    solve_and_check(csr, matrix_rows, expected)


@pytest.mark.parametrize("mode", ["wavefront", "sync_free"])
@pytest.mark.parametrize("band_width", [2, 5, 64])
def test_band_chains_run_in_both_executors(oracle, band_width, mode):
    """band_width > 1: one task per connected component of a band of levels,
    members in sequence; fewer launches (level launches) or a poll per chain
    member (persistent executor, on dependence counters), same results."""
    print("band chains", band_width, mode, flush=True)
    csc = sptrsv.compile_sptrsv_csc(execution_mode=mode,
                                    threads_per_block=128, task_lanes=4,
                                    band_width=band_width)
    csr = sptrsv.compile_sptrsv_csr(execution_mode=mode,
                                    threads_per_block=128, task_lanes=8,
                                    band_width=band_width)
    lane = sptrsv.compile_sptrsv_csc(execution_mode="wavefront",
                                     threads_per_block=64, thread_map=None,
                                     band_width=band_width)
    for name, overrides in (("c1", {}), ("c2", dict(nx=20, ny=18, nz=16)),
                            ("c5", dict(n=3000))):
        work = workloads.configuration(name, **overrides)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(csc, work, expected)
        solve_and_check(lane, work, expected)
    assert "task_ptr[_task + 1]" in csc.hip_kernel_source
    assert csc.hip_lowering.dependence_protocol == "counter"
    assert csc.hip_lowering.tile_rows is None
    work = workloads.configuration("c3", n=20000)
    expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solve_and_check(csr, work, expected)
    factor = spilu0.compile_ilu0_csr(execution_mode=mode,
                                     threads_per_block=128, task_lanes=8,
                                     thread_unroll=1, band_width=band_width)
    work = workloads.configuration("c4", nx=40, ny=36)
    expected = oracle.ilu0_csr(work.data, work.indices, work.indptr)
    np.testing.assert_array_equal(
        factor(work.data.copy(), work.indices, work.indptr), expected)
    assert factor.hip_lowering.dependence_protocol == "counter"
    if mode == "sync_free":
        # a whole workgroup per task cannot walk a chain member by member
        with pytest.raises(Exception, match="one wavefront or less"):
            sptrsv.compile_sptrsv_csc(
                execution_mode="sync_free", threads_per_block=128, n_warp=2,
                band_width=band_width)(work.indptr, work.indices, work.data,
                                       np.ones(work.n), work.n)


ILU_VARIANTS = [
    dict(execution_mode="wavefront", threads_per_block=128, thread_unroll=1),
    dict(execution_mode="wavefront", threads_per_block=128, task_lanes=4),
    dict(execution_mode="wavefront", threads_per_block=128, task_lanes=8,
         thread_unroll=2),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=8),
    dict(execution_mode="sync_free", threads_per_block=128, n_warp=1),
    dict(execution_mode="wavefront", threads_per_block=128, n_warp=2),
    dict(execution_mode=None, threads_per_block=None),
    # the task waits for its pivot rows one by one
    dict(execution_mode="sync_free", threads_per_block=64, task_lanes=8,
         dependence_protocol="pull"),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=1,
         dependence_protocol="pull"),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=64,
         dependence_protocol="pull", segment_cache=False),
    # one row per wavefront: final values published, polled by the readers
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=64,
         dependence_protocol="pull"),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=64,
         dependence_protocol="pull", publish_values=False),
    # published values in tiles: a workgroup owns consecutive rows and keeps
    # their slice of the publication buffer in LDS (tiles that are not whole
    # grid lines; a copy too small for a tile, which then runs without it)
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=64,
         dependence_protocol="pull", tile_rows=100, tile_positions=1024,
         segment_capacity=64),
    dict(execution_mode="sync_free", threads_per_block=64, task_lanes=64,
         dependence_protocol="pull", tile_rows=72, tile_positions=700),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=64,
         dependence_protocol="pull", tile_rows=256, tile_positions=512),
    # the own row staged in LDS although it would fit the registers
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=64,
         dependence_protocol="pull", segment_registers=False),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=64,
         dependence_protocol="pull", tile_rows=100, tile_positions=1024,
         segment_registers=False),
]


@pytest.mark.parametrize("options", ILU_VARIANTS, ids=lambda o: "-".join(
    f"{k}={v}" for k, v in o.items()))
def test_ilu0_csr_variants(oracle, options):
    print("ilu0", options, flush=True)
    factor = spilu0.compile_ilu0_csr(**options)
    work = workloads.configuration("c4", nx=72, ny=56)
    expected = oracle.ilu0_csr(work.data, work.indices, work.indptr)
    original = work.data.copy()
    result = factor(work.data.copy(), work.indices, work.indptr)
    np.testing.assert_array_equal(work.data, original)
    # every entry is updated once per pivot, by one lane, in ascending pivot
    # order: the evaluation order is the sequential loop's
    np.testing.assert_array_equal(result, expected)
    assert len(factor.structural_lookups) == 1
    assert factor.structural_lookups[0].name in factor.hip_kernel_source
    assert "for (diag_ptr" not in factor.hip_kernel_source
    if options.get("dependence_protocol") == "pull":
        assert factor.hip_lowering.dependence_protocol == "pull"
        assert "_lcd_blocked" in factor.hip_kernel_source
        published = (options["task_lanes"] == 64
                     and options.get("segment_cache", True)
                     and options.get("publish_values", True))
        assert ("_lcd_pub" in factor.hip_kernel_source) == published
        if "tile_rows" in options:
            assert factor.hip_lowering.tile_rows == options["tile_rows"]
            assert "_lcd_ptile[LCD_TILE_POS]" in factor.hip_kernel_source
        assert ("done[" in factor.hip_kernel_source) != published
        # rows of at most 64 entries live in registers, one entry per lane
        registers = published and options.get("segment_registers", True)
        assert factor.hip_lowering.segment_registers == registers
        assert ("lcd_rseg_uni(_lcd_rseg" in factor.hip_kernel_source) == registers
        # irregular rows too: pivots near and far, empty lower parts
        import scipy.sparse as sp
        lower, diagonal, _ = random_lower_factor(2500, 11)
        matrix = sp.csr_matrix(lower + lower.T * 0.5 + sp.diags(4 * diagonal))
        matrix.sort_indices()
        indptr = matrix.indptr.astype(np.int32)
        indices = matrix.indices.astype(np.int32)
        np.testing.assert_array_equal(
            factor(matrix.data.copy(), indices, indptr),
            oracle.ilu0_csr(matrix.data, indices, indptr))
        # (rows of up to 300 entries: staged in LDS or updated in place)
        assert not factor.hip_lowering.segment_registers
        if published:
            forced = spilu0.compile_ilu0_csr(**{**options,
                                                "segment_registers": True})
            with pytest.raises(ValueError, match="at most 64"):
                forced(matrix.data.copy(), indices, indptr)


def test_ilu0_level_launches_with_the_row_in_registers(oracle):
    """ILU0 under level launches, a row per wavefront: the task of the
    persistent pull executor (row in registers, pivot searches in the
    inspector's tables, the next pivot located ahead) with plain loads --
    every pivot row was finished by an earlier launch.  Bit-identical on the
    stencil and on rows of uneven length; a structure with rows beyond 64
    entries keeps the counters and the searches."""
    print("ilu0 level pull", flush=True)
    factor = spilu0.compile_ilu0_csr(
        execution_mode="wavefront", threads_per_block=128, task_lanes=64,
        thread_unroll=1, dependence_protocol="pull")
    work = workloads.configuration("c4", nx=72, ny=56)
    expected = oracle.ilu0_csr(work.data, work.indices, work.indptr)
    for _ in range(2):
        np.testing.assert_array_equal(
            factor(work.data.copy(), work.indices, work.indptr), expected)
    lowering = factor.hip_lowering
    assert lowering.execution_mode == "wavefront"
    assert lowering.dependence_protocol == "pull" and lowering.segment_registers
    source = factor.hip_kernel_source
    assert "_lcd_pair[" in source and "lcd_sorted_find" not in source
    assert "_lcd_pub" not in source and "lcd_pull_settle(" not in source
    # (the first four pivots of a row are taken flat, the pivot loop has the
    # rest: the random rows below have up to a dozen)
    assert "_f3__sp_kj_ptr_o = _lcd_pair[" in source
    assert "for (; k_ptr < _lcd_low_end; ++k_ptr) {" in source
    import scipy.sparse as sp
    rng = np.random.default_rng(5)
    n = 3000
    pattern = sp.random(n, n, density=6.0 / n, random_state=3, format="csr")
    pattern = pattern + pattern.T + sp.identity(n)
    matrix = sp.csr_matrix(pattern)
    matrix.data = rng.uniform(-1.0, 1.0, len(matrix.data))
    matrix = sp.csr_matrix(matrix + sp.diags(np.full(n, 40.0)))
    matrix.sort_indices()
    assert np.diff(matrix.indptr).max() <= 64
    indptr = matrix.indptr.astype(np.int32)
    indices = matrix.indices.astype(np.int32)
    np.testing.assert_array_equal(
        factor(matrix.data.copy(), indices, indptr),
        oracle.ilu0_csr(matrix.data, indices, indptr))
    assert factor.hip_lowering.segment_registers
    lower, diagonal, _ = random_lower_factor(2500, 11)
    long_rows = sp.csr_matrix(lower + lower.T * 0.5 + sp.diags(4 * diagonal))
    long_rows.sort_indices()
    indptr = long_rows.indptr.astype(np.int32)
    indices = long_rows.indices.astype(np.int32)
    np.testing.assert_array_equal(
        factor(long_rows.data.copy(), indices, indptr),
        oracle.ilu0_csr(long_rows.data, indices, indptr))
    assert not factor.hip_lowering.segment_registers
    assert factor.hip_lowering.dependence_protocol == "counter"


@pytest.mark.parametrize("mode", ["wavefront", "sync_free", None])
def test_ilu0_csc_matches_the_sequential_loop(oracle, mode):
    """compiler/e2e_tests/test_spilu0_e2e.py:107-121: the column form, every
    column after all earlier ones, one thread per column; the operation
    order is the sequential loop's, so the factor is bit-identical."""
    from scipy.sparse import csc_matrix, csr_matrix
    print("ilu0 csc", mode, flush=True)
    rng = np.random.default_rng(21)
    n = 150
    pattern = (rng.random((n, n)) < 5.0 / n) | np.eye(n, dtype=bool)
    a = np.where(pattern, rng.uniform(-1, 1, (n, n)), 0.0) + 8 * np.eye(n)
    a[40, 40] = 0.0                      # a pivot that stays zero is skipped
    a[:40, 40] = a[40, :40] = 0.0
    matrix = csc_matrix(a)
    matrix.sort_indices()
    indptr = matrix.indptr.astype(np.int32)
    indices = matrix.indices.astype(np.int32)
    factor = spilu0.compile_ilu0_csc(execution_mode=mode)
    expected = oracle.ilu0_csc(matrix.data, indices, indptr)
    original = matrix.data.copy()
    result = factor(matrix.data.copy(), indices, indptr)
    np.testing.assert_array_equal(matrix.data, original)
    np.testing.assert_array_equal(result, expected)
    dag, _ = factor.build_dag(matrix.data, indices, indptr)
    assert dag == [list(range(k + 1, n)) for k in range(n)]
    # the row form of the same matrix gives the same incomplete factor
    by_row = csr_matrix(matrix)
    by_row.sort_indices()
    row_factor = spilu0.compile_ilu0_csr(execution_mode="wavefront")(
        by_row.data.copy(), by_row.indices.astype(np.int32),
        by_row.indptr.astype(np.int32))
    np.testing.assert_allclose(
        csc_matrix((result, indices, indptr), shape=a.shape).toarray(),
        csr_matrix((row_factor, by_row.indices, by_row.indptr),
                   shape=a.shape).toarray(), rtol=1e-12, atol=1e-14)


def test_ilu0_dense_pattern_is_lu(oracle):
    """On a dense pattern ILU0 is LU without pivoting."""
    rng = np.random.default_rng(5)
    n = 24
    dense = rng.uniform(-1, 1, (n, n)) + n * np.eye(n)
    indptr = np.arange(0, n * n + 1, n, dtype=np.int32)
    indices = np.tile(np.arange(n, dtype=np.int32), n)
    factor = spilu0.compile_ilu0_csr(execution_mode="sync_free",
                                     threads_per_block=128, task_lanes=8)
    result = factor(dense.ravel().copy(), indices, indptr).reshape(n, n)
    lower = np.tril(result, -1) + np.eye(n)
    upper = np.triu(result)
    np.testing.assert_allclose(lower @ upper, dense, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("n,capacity", [(24, None), (48, 32), (150, 32),
                                        (150, None)])
def test_ilu0_published_values_on_long_rows(oracle, n, capacity):
    """Rows that fit the staged segment, rows that are updated in place and
    read back for publication (a small staging capacity forces that path),
    rows longer than a wavefront; the same bound call factorises three
    matrices in a row."""
    rng = np.random.default_rng(n)
    indptr = np.arange(0, n * n + 1, n, dtype=np.int32)
    indices = np.tile(np.arange(n, dtype=np.int32), n)
    factor = spilu0.compile_ilu0_csr(execution_mode="sync_free",
                                     threads_per_block=128, task_lanes=64,
                                     dependence_protocol="pull",
                                     segment_capacity=capacity)
    for launch in range(3):
        dense = rng.uniform(-1, 1, (n, n)) + n * np.eye(n)
        result = factor(dense.ravel().copy(), indices, indptr)
        assert "_lcd_pub" in factor.hip_kernel_source
        np.testing.assert_array_equal(
            result, oracle.ilu0_csr(dense.ravel(), indices, indptr))
        result = result.reshape(n, n)
        lower = np.tril(result, -1) + np.eye(n)
        np.testing.assert_allclose(lower @ np.triu(result), dense,
                                   rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed,tiles", [(1, None), (2, 300), (3, None)])
def test_ilu0_irregular_rows_in_registers(oracle, seed, tiles):
    """Rows in registers and searches from the inspector's tables on a
    structure that is no stencil: unsymmetric random pattern with rows of 0 to
    30 entries, rows without a diagonal entry (the pivot is skipped), exact
    zeros on the diagonal (skipped as well), pivot rows that lack most of the
    columns a row holds; the same plan factorises two sets of values."""
    import scipy.sparse as sp
    print("irregular ilu0", seed, tiles, flush=True)
    rng = np.random.default_rng(seed)
    n = 4000
    rows, cols = [], []
    for i in range(n):
        count = int(rng.integers(0, 25))
        near = rng.integers(max(0, i - 60), min(n, i + 60), size=count)
        far = rng.integers(0, n, size=count // 6)
        picks = set(np.concatenate([near, far]).tolist())
        if rng.random() < 0.9:
            picks.add(i)              # most rows have their diagonal entry
        picks = sorted(picks)[:64]
        rows += [i] * len(picks)
        cols += picks
    values = rng.uniform(-1.0, 1.0, len(rows))
    matrix = sp.csr_matrix((values, (rows, cols)), shape=(n, n))
    matrix.sort_indices()
    indptr = matrix.indptr.astype(np.int32)
    indices = matrix.indices.astype(np.int32)
    assert np.diff(indptr).max() <= 64 and np.diff(indptr).min() == 0
    factor = spilu0.compile_ilu0_csr(
        execution_mode="sync_free", threads_per_block=256, task_lanes=64,
        dependence_protocol="pull",
        **({"tile_rows": tiles, "tile_positions": 8192} if tiles else {}))
    for launch in range(2):
        data = rng.uniform(-1.0, 1.0, len(values))
        diagonal = indices == np.repeat(np.arange(n), np.diff(indptr))
        data[diagonal] += 8.0 * np.sign(data[diagonal])
        # exact zeros on some diagonals: those pivots are left alone
        data[np.nonzero(diagonal)[0][::17]] = 0.0
        expected = oracle.ilu0_csr(data.copy(), indices, indptr)
        assert np.all(np.isfinite(expected))
        result = factor(data.copy(), indices, indptr)
        np.testing.assert_array_equal(result, expected)
    plan = factor.schedule_plan(data, indices, indptr)
    assert plan.segment_registers == 2
    assert factor.hip_lowering.segment_registers
    assert factor.hip_lowering.structure_tables
    assert "lcd_sorted_find(" not in factor.hip_kernel_source
    # the same structure with the searches left in the kernel, and with the
    # rows staged in LDS: the same bits
    for options in (dict(pair_tables=False), dict(segment_registers=False)):
        other = spilu0.compile_ilu0_csr(
            execution_mode="sync_free", threads_per_block=128, task_lanes=64,
            dependence_protocol="pull", **options)
        np.testing.assert_array_equal(other(data.copy(), indices, indptr),
                                      expected)
        assert other.schedule_plan(data, indices, indptr).segment_registers == (
            1 if "pair_tables" in options else 0)


def ilu0_own_diagonal(A_data, A_indices, A_indptr):
    """ILU0 whose updates are scaled by the row's own diagonal entry as it
    stands at that pivot: a read of the task's own row at a position that is
    searched for, not walked by a loop."""
    n = len(A_indptr) - 1
    for i in range(n):
        row_start = A_indptr[i]
        row_end = A_indptr[i + 1]
        for k_ptr in range(row_start, row_end):
            k = A_indices[k_ptr]
            if k >= i:
                break
            diag_val = 0.0
            for diag_ptr in range(A_indptr[k], A_indptr[k + 1]):
                if A_indices[diag_ptr] == k:
                    diag_val = A_data[diag_ptr]
                    break
            own = 1.0
            for own_ptr in range(A_indptr[i], A_indptr[i + 1]):
                if A_indices[own_ptr] == i:
                    own = A_data[own_ptr]
                    break
            if diag_val != 0.0:
                A_data[k_ptr] = A_data[k_ptr] / diag_val
                l_ik = A_data[k_ptr]
                for j_ptr in range(k_ptr + 1, row_end):
                    j = A_indices[j_ptr]
                    for kj_ptr in range(A_indptr[k], A_indptr[k + 1]):
                        if A_indices[kj_ptr] == j:
                            u_kj = A_data[kj_ptr]
                            A_data[j_ptr] = (
                                A_data[j_ptr] - l_ik * u_kj * own
                            )
                            break
    return A_data


@pytest.mark.parametrize("registers", [True, False])
def test_own_row_read_at_a_searched_position(registers):
    """With the own row in registers, a read of it at a computed position
    goes to the write-only copy in LDS and sees every update made so far;
    against the loop itself run by CPython."""
    from lcd_amd import parallel
    print("own row at a searched position", registers, flush=True)
    work = workloads.configuration("c4", nx=24, ny=20)
    rng = np.random.default_rng(9)
    data = work.data * rng.uniform(0.05, 0.1, len(work.data))
    diagonal = work.indices == np.repeat(np.arange(work.n),
                                         np.diff(work.indptr))
    data[diagonal] = rng.uniform(1.0, 1.5, int(diagonal.sum()))
    expected = ilu0_own_diagonal(data.copy(), work.indices, work.indptr)
    assert np.all(np.isfinite(expected))
    factor = parallel(
        block_map="i", thread_map="j_ptr",
        function_props=spilu0.FUNCTION_PROPS, execution_mode="sync_free",
        threads_per_block=128, task_lanes=64, thread_unroll=1,
        dependence_protocol="pull",
        segment_registers=registers)(ilu0_own_diagonal)
    for _ in range(2):
        result = factor(data.copy(), work.indices, work.indptr)
        np.testing.assert_array_equal(result, expected)
    assert factor.hip_lowering.segment_registers == registers
    assert len(factor.structural_lookups) == 1
    if registers:
        assert ("own = lcd_rseg_ldp(_lcd_pub, _lcd_seg, _lcd_seg_base, "
                "_lcd_seg_own, own_ptr") in factor.hip_kernel_source


@pytest.mark.parametrize("variant", ["simple", "full"])
def test_gauss_seidel_two_sweeps(oracle, variant):
    from scipy.sparse import csr_matrix
    work = workloads.configuration("c4", nx=40, ny=32)
    matrix = csr_matrix((work.data, work.indices, work.indptr),
                        shape=(work.n, work.n))
    rng = np.random.default_rng(9)
    rhs, start = rng.random(work.n), rng.random(work.n)
    if variant == "simple":
        from scipy.sparse import tril
        strict = tril(matrix, -1, format="csr")
        strict.sort_indices()
        diagonal = matrix.diagonal()
        ap = strict.indptr.astype(np.int32)
        ai = strict.indices.astype(np.int32)
        expected = oracle.gauss_seidel_csr(ap, ai, strict.data, diagonal, rhs,
                                           start, work.n, 2)
        result = gauss_seidel.simple_gauss_seidel_csr(
            ap, ai, strict.data, diagonal, rhs, start.copy(), work.n, 2)
        np.testing.assert_array_equal(result, expected)
    else:
        lower = csr_matrix(np.tril(matrix.toarray()))
        lower.sort_indices()
        ap = lower.indptr.astype(np.int32)
        ai = lower.indices.astype(np.int32)
        expected = start.copy()
        for _ in range(2):
            for i in range(work.n):
                sigma, diag = 0.0, 1.0
                for j in range(ap[i], ap[i + 1]):
                    if ai[j] == i:
                        diag = lower.data[j]
                    else:
                        sigma += lower.data[j] * expected[ai[j]]
                expected[i] = (rhs[i] - sigma) / diag
        result = gauss_seidel.full_gauss_seidel_csr(
            ap, ai, lower.data, rhs, start.copy(), work.n, 2)
        np.testing.assert_array_equal(result, expected)


def band_factor(n, offsets_per_column, seed, diagonal=(0.5, 2.0)):
    """Lower-triangular CSC factor whose column i holds the diagonal first and
    then rows i + d for a random subset of the distances d in 1 .. span."""
    rng = np.random.default_rng(seed)
    span, keep = offsets_per_column
    indptr, indices, data = [0], [], []
    for i in range(n):
        distances = np.arange(1, min(span, n - 1 - i) + 1)
        if keep < 1.0 and len(distances):
            distances = distances[rng.random(len(distances)) < keep]
        indices.append(i)
        data.append(rng.uniform(*diagonal))
        indices.extend((i + distances).tolist())
        data.extend(rng.uniform(-0.3, 0.3, len(distances)).tolist())
        indptr.append(len(indices))
    return (np.asarray(indptr, dtype=np.int32),
            np.asarray(indices, dtype=np.int32), np.asarray(data))


WALKER = dict(execution_mode="sync_free", dependence_protocol="mailbox",
              task_lanes=4, band_walker=True)


@pytest.mark.parametrize("n,span,keep,tpb", [
    (2, 1, 1.0, 128), (50, 3, 1.0, 128), (64, 8, 1.0, 256), (65, 1, 1.0, 128),
    (129, 63, 1.0, 1024), (1000, 8, 1.0, None), (4113, 63, 0.3, 512),
    (5000, 40, 0.1, None), (3000, 63, 1.0, 256)])
def test_band_walker(oracle, n, span, keep, tpb):
    """One wavefront runs the tasks in program order: results are the
    sequential loop's bit for bit, whatever the block boundaries (n below,
    at and off multiples of 64), the band (1 to 63, full or sparse) and the
    number of wavefronts that stage for the walker."""
    print("band walker", n, span, keep, tpb, flush=True)
    options = dict(WALKER)
    if tpb:
        options["threads_per_block"] = tpb
    solver = sptrsv.compile_sptrsv_csc(**options)
    indptr, indices, data = band_factor(n, (span, keep), seed=n + span)
    rhs = np.random.default_rng(n).standard_normal(n)
    expected = oracle.sptrsv_csc(indptr, indices, data, rhs, n)
    for _ in range(2):       # the second call replays the captured graph
        result = solver(indptr, indices, data, rhs, n)
        np.testing.assert_array_equal(result, expected)
    plan = solver.schedule_plan(indptr, indices, data, rhs, n)
    assert plan.band_walker and plan.tile_rows is None
    assert solver.hip_lowering.band_walker
    assert "lcd_div_prepare(" in solver.hip_kernel_source
    assert plan.schedule.threads_per_block == (tpb or 1024)


@pytest.mark.parametrize("n,span,keep,tpb", [
    (3, 2, 1.0, 128), (64, 8, 1.0, 256), (130, 63, 1.0, None),
    (1000, 8, 1.0, None), (4113, 63, 0.3, 512), (5000, 40, 0.1, None)])
def test_band_walker_csr(oracle, n, span, keep, tpb):
    """The pull-shaped solve on the walker: a task's element starts as b[i]
    (staged per task, taken by the lane with the task), the row's products
    are subtracted as their sources finish, the division by the diagonal
    ends it -- the sequential loop's order, so bit for bit its result (the
    other CSR executors sum a row's products first)."""
    import scipy.sparse as sp
    print("band walker, CSR", n, span, keep, tpb, flush=True)
    indptr, indices, data = band_factor(n, (span, keep), seed=2 * n + span)
    lower = sp.csc_matrix((data, indices, indptr), shape=(n, n)).tocsr()
    lower.sort_indices()
    rp, ci = lower.indptr.astype(np.int32), lower.indices.astype(np.int32)
    rhs = np.random.default_rng(n + 1).standard_normal(n)
    options = dict(execution_mode="sync_free", dependence_protocol="pull",
                   task_lanes=8, band_walker=True)
    if tpb:
        options["threads_per_block"] = tpb
    solver = sptrsv.compile_sptrsv_csr(**options)
    expected = sptrsv.sptrsv_csr_loop(rp, ci, lower.data, rhs, n)
    for _ in range(2):
        result = solver(rp, ci, lower.data, rhs, n)
        np.testing.assert_array_equal(result, expected)
    assert relative_error(result, oracle.sptrsv_csr(rp, ci, lower.data, rhs,
                                                    n)) <= TOLERANCE
    plan = solver.schedule_plan(rp, ci, lower.data, rhs, n)
    assert plan.band_walker and solver.hip_lowering.band_walker
    # values the prepared reciprocal does not cover: the second pass
    rhs[n // 2] = 0.0 if n < 200 else np.inf
    with np.errstate(all="ignore"):
        expected = sptrsv.sptrsv_csr_loop(rp, ci, lower.data, rhs, n)
    np.testing.assert_array_equal(solver(rp, ci, lower.data, rhs, n), expected)
    # an element that starts as -0.0 keeps its sign through the empty cells
    # of the table (rows whose sources are all zero: the result is -0.0 / d)
    rhs = np.zeros(n)
    rhs[::3] = -0.0
    with np.errstate(all="ignore"):
        expected = sptrsv.sptrsv_csr_loop(rp, ci, lower.data, rhs, n)
    result = solver(rp, ci, lower.data, rhs, n)
    np.testing.assert_array_equal(result, expected)
    np.testing.assert_array_equal(np.signbit(result), np.signbit(expected))
    assert np.any(np.signbit(expected))
    # chosen by itself for a chain in CSR form, not for a power-law matrix
    auto = sptrsv.compile_sptrsv_csr(execution_mode="sync_free",
                                     dependence_protocol="pull", task_lanes=8)
    if keep == 1.0:
        assert auto.schedule_plan(rp, ci, lower.data, rhs, n).band_walker
    grid = workloads.configuration("c3", n=2000)
    assert not auto.schedule_plan(grid.indptr, grid.indices, grid.data,
                                  grid.rhs, grid.n).band_walker


def test_band_walker_divides_again_where_the_prepared_reciprocal_does_not_apply(
        oracle):
    """Zero, tiny, huge and non-finite numerators and divisors: the blocks
    they fall in run a second time with the general division (and with the
    products of real edges only, so 0 * inf of a missing edge never shows);
    an explicitly stored zero coefficient still gives 0 * inf = NaN as in
    the sequential loop."""
    n = 1000
    indptr, indices, data = band_factor(n, (8, 1.0), seed=3)
    solver = sptrsv.compile_sptrsv_csc(**WALKER)
    rng = np.random.default_rng(11)
    cases = {}
    rhs = rng.standard_normal(n)
    rhs[:130] = 0.0                      # exact zeros: x = 0 over two blocks
    cases["zeros"] = (data.copy(), rhs)
    rhs = rng.standard_normal(n)
    rhs[200] = 1e-305                    # quotient far down the range
    rhs[400] = 1e300
    cases["range"] = (data.copy(), rhs)
    values = data.copy()
    values[indptr[300]] = 1e-200         # divisors the sequence scales
    values[indptr[301]] = 1e250
    values[indptr[500]] = 5e-324
    cases["divisors"] = (values, rng.standard_normal(n))
    rhs = rng.standard_normal(n)
    rhs[600] = np.inf
    rhs[900] = np.nan
    cases["not finite"] = (data.copy(), rhs)
    values = data.copy()
    values[indptr[700]] = 0.0            # x[700] = b / 0
    values[indptr[700] + 3] = 0.0        # ... times a stored zero: NaN
    cases["zero pivot"] = (values, rng.standard_normal(n))
    for name, (values, rhs) in cases.items():
        print("band walker,", name, flush=True)
        with np.errstate(all="ignore"):
            expected = oracle.sptrsv_csc(indptr, indices, values, rhs, n)
        result = solver(indptr, indices, values, rhs, n)
        np.testing.assert_array_equal(result, expected, err_msg=name)
        # (also the signs of zeros; the sign of a NaN is the machine's)
        valid = ~np.isnan(expected)
        np.testing.assert_array_equal(np.signbit(result[valid]),
                                      np.signbit(expected[valid]), err_msg=name)


def test_band_walker_is_chosen_for_chains_only(oracle):
    """The automatic choice: close to one task per level and every edge
    shorter than 64 iterations."""
    solver = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                       dependence_protocol="mailbox",
                                       task_lanes=4)
    chain = workloads.configuration("c5", n=3000)
    grid = workloads.configuration("c1")
    wide = band_factor(2000, (64, 1.0), seed=5)      # one edge too long
    forks = band_factor(4000, (12, 0.02), seed=6)    # many tasks per level
    for work, walks in ((chain, True), (grid, False)):
        plan = solver.schedule_plan(work.indptr, work.indices, work.data,
                                    work.rhs, work.n)
        assert plan.band_walker == walks
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(solver, work, expected, exact=True)
    for (indptr, indices, data), n in ((wide, 2000), (forks, 4000)):
        rhs = np.ones(n)
        plan = solver.schedule_plan(indptr, indices, data, rhs, n)
        assert not plan.band_walker
        np.testing.assert_array_equal(
            solver(indptr, indices, data, rhs, n),
            oracle.sptrsv_csc(indptr, indices, data, rhs, n))
    # a chain long enough for the estimates to matter: the plan runs on the
    # walker and says that one host core would be faster
    from lcd_amd.scheduler import SchedulerAdvice
    long_chain = workloads.configuration("c5", n=40000)
    fresh = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                      dependence_protocol="mailbox",
                                      task_lanes=4)
    with pytest.warns(SchedulerAdvice, match="close to a chain"):
        plan = fresh.schedule_plan(long_chain.indptr, long_chain.indices,
                                   long_chain.data, long_chain.rhs,
                                   long_chain.n)
    assert plan.band_walker and "host core" in plan.advice
    assert solver.schedule_plan(grid.indptr, grid.indices, grid.data,
                                grid.rhs, grid.n).advice is None
    never = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                      dependence_protocol="mailbox",
                                      task_lanes=4, band_walker=False)
    assert not never.schedule_plan(chain.indptr, chain.indices, chain.data,
                                   chain.rhs, chain.n).band_walker
    # a workgroup of one wavefront has nobody to stage for the walker
    single = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                       dependence_protocol="mailbox",
                                       task_lanes=4, threads_per_block=64)
    assert not single.schedule_plan(chain.indptr, chain.indices, chain.data,
                                    chain.rhs, chain.n).band_walker
    solve_and_check(single, chain, oracle.sptrsv_csc(
        chain.indptr, chain.indices, chain.data, chain.rhs, chain.n),
        exact=True)
    with pytest.raises(Exception, match="two wavefronts"):
        sptrsv.compile_sptrsv_csc(threads_per_block=64, **WALKER)(
            chain.indptr, chain.indices, chain.data, chain.rhs, chain.n)
    forced = sptrsv.compile_sptrsv_csc(**WALKER)
    with pytest.raises(ValueError, match="fewer than 64 iterations"):
        forced(wide[0], wide[1], wide[2], np.ones(2000), 2000)
    # asked for by name it also runs a DAG with many tasks per level
    indptr, indices, data = forks
    np.testing.assert_array_equal(
        forced(indptr, indices, data, np.ones(4000), 4000),
        oracle.sptrsv_csc(indptr, indices, data, np.ones(4000), 4000))


def test_band_walker_refuses_a_repeated_edge():
    """Two entries of one column with the same row index are two edges
    between the same two tasks; the walker's table has one cell for them and
    says so instead of returning a wrong result."""
    from lcd_amd import hip_runtime
    n = 200
    indptr, indices, data = band_factor(n, (4, 1.0), seed=9)
    indices = indices.copy()
    indices[indptr[50] + 2] = indices[indptr[50] + 1]
    # asked for by name: refused on the host, before anything is launched
    solver = sptrsv.compile_sptrsv_csc(**WALKER)
    with pytest.raises(ValueError, match="band_walker=True"):
        solver(indptr, indices, data, np.ones(n), n)
    # left to the scheduler: the structure keeps an executor that takes
    # every entry, and the result is the sequential loop's
    from oracle import lcd_oracle
    automatic = sptrsv.compile_sptrsv_csc(
        **{key: value for key, value in WALKER.items() if key != "band_walker"})
    result = automatic(indptr, indices, data, np.ones(n), n)
    plan = automatic.schedule_plan(indptr, indices, data, np.ones(n), n)
    assert not plan.band_walker
    expected = lcd_oracle.sptrsv_csc(indptr, indices, data, np.ones(n), n)
    assert elementwise_error(result, expected) <= TOLERANCE


def walker_unit_lower(Ap, Ai, Ax, b, n):
    x = np.zeros(n)
    for i in range(n):
        x[i] = b[i] - x[i]
        for j in range(Ap[i] + 1, Ap[i + 1]):
            x[Ai[j]] += Ax[j] * x[i]
    return x


def walker_subtracting(Ap, Ai, Ax, b, n):
    x = np.zeros(n)
    for i in range(n):
        x[i] = (b[i] + x[i]) / Ax[Ap[i]] + 0.5 * b[i]
        for j in range(Ap[i] + 1, Ap[i + 1]):
            x[Ai[j]] -= x[i] * Ax[j]
    return x


@pytest.mark.parametrize("loop", [walker_unit_lower, walker_subtracting])
def test_band_walker_other_loops(loop):
    """Loops of the same form with no division at all, with a division that
    is not the task's value, and with products that are subtracted, against
    the loop itself run by CPython."""
    from lcd_amd import parallel
    solver = parallel(block_map="i", thread_map="j",
                      function_props=sptrsv.FUNCTION_PROPS_CSC, **WALKER)(loop)
    n = 700
    indptr, indices, data = band_factor(n, (9, 0.7), seed=21)
    rhs = np.random.default_rng(4).standard_normal(n)
    expected = loop(indptr, indices, data, rhs, n)
    result = solver(indptr, indices, data, rhs, n)
    np.testing.assert_array_equal(result, expected)
    assert solver.hip_lowering.band_walker
    assert ("lcd_div_prepare(" in solver.hip_kernel_source) == (
        loop is walker_subtracting)


def test_level_walker(oracle):
    """Small DAGs with narrow levels run on one wavefront, a level per step,
    values in LDS: no poll, the sequential loop's arithmetic, bit for bit --
    for the push-shaped solve (CSC) and the pull-shaped one (CSR, against the
    loop itself run by CPython)."""
    import scipy.sparse as sp
    walker = dict(execution_mode="sync_free", task_lanes=4, level_walker=True)
    csc = sptrsv.compile_sptrsv_csc(dependence_protocol="mailbox", **walker)
    csr = sptrsv.compile_sptrsv_csr(dependence_protocol="pull", **walker)
    cases = [workloads.configuration("c1"),
             workloads.configuration("c1", nx=37, ny=11),
             workloads.configuration("c2", nx=6, ny=5, nz=7),
             workloads.configuration("c2", nx=16, ny=16, nz=16),
             workloads.configuration("c5", n=300, bandwidth=3)]
    for work in cases:
        print("level walker", work.name, flush=True)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        for _ in range(2):
            solve_and_check(csc, work, expected, exact=True)
        plan = csc.schedule_plan(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
        assert plan.level_walker >= 1 and csc.hip_lowering.level_walker
        assert "lcd_ld" not in csc.hip_kernel_source
        lower = sp.csc_matrix((work.data, work.indices, work.indptr),
                              shape=(work.n, work.n)).tocsr()
        lower.sort_indices()
        rp = lower.indptr.astype(np.int32)
        ci = lower.indices.astype(np.int32)
        np.testing.assert_array_equal(
            csr(rp, ci, lower.data, work.rhs, work.n),
            sptrsv.sptrsv_csr_loop(rp, ci, lower.data, work.rhs, work.n))
        assert csr.hip_lowering.level_walker
    # values that are not finite, zeros and their signs
    work = cases[1]
    rhs = work.rhs.copy()
    rhs[5], rhs[40], rhs[100:140] = np.inf, -0.0, 0.0
    with np.errstate(all="ignore"):
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     rhs, work.n)
    result = csc(work.indptr, work.indices, work.data, rhs, work.n)
    np.testing.assert_array_equal(result, expected)
    valid = ~np.isnan(expected)
    np.testing.assert_array_equal(np.signbit(result[valid]),
                                  np.signbit(expected[valid]))
    # divisors and quotients the prepared reciprocal does not serve: their
    # blocks run again with the general division
    values = work.data.copy()
    values[work.indptr[50]] = 1e-200
    values[work.indptr[51]] = 1e250
    values[work.indptr[200]] = 5e-324
    rhs = work.rhs.copy()
    rhs[300] = 1e-305
    with np.errstate(all="ignore"):
        expected = oracle.sptrsv_csc(work.indptr, work.indices, values, rhs,
                                     work.n)
    np.testing.assert_array_equal(
        csc(work.indptr, work.indices, values, rhs, work.n), expected)
    # chosen by itself for such a DAG; not for one with wide levels, too many
    # tasks, or too many incoming entries per task (then the tiles)
    auto = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                     dependence_protocol="mailbox",
                                     task_lanes=4)
    for work, walks in ((cases[0], True),
                        (workloads.configuration("c1", nx=80, ny=80), False),
                        # levels of up to 100 tasks: two steps each
                        (workloads.configuration("c2", nx=15, ny=15, nz=15),
                         True),
                        (workloads.configuration("c5", n=3000), False)):
        plan = auto.schedule_plan(work.indptr, work.indices, work.data,
                                  work.rhs, work.n)
        assert bool(plan.level_walker) == walks, work.name
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(auto, work, expected, exact=True)
    with pytest.raises(ValueError, match="level_walker=True needs"):
        big = workloads.configuration("c1", nx=80, ny=80)
        csc(big.indptr, big.indices, big.data, big.rhs, big.n)
    never = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                      dependence_protocol="mailbox",
                                      task_lanes=4, level_walker=False)
    first = cases[0]
    assert not never.schedule_plan(first.indptr, first.indices, first.data,
                                   first.rhs, first.n).level_walker


def test_edge_cases(oracle):
    solver = sptrsv.compile_sptrsv_csc(execution_mode="sync_free",
                                       threads_per_block=128, task_lanes=4)
    # a single unknown
    x = solver(np.array([0, 1], dtype=np.int32), np.array([0], dtype=np.int32),
               np.array([2.0]), np.array([3.0]), 1)
    assert x.tolist() == [1.5]
    # diagonal matrix: no edges, one level
    n = 1000
    diag = np.linspace(1.0, 2.0, n)
    rhs = np.arange(n, dtype=np.float64)
    x = solver(np.arange(n + 1, dtype=np.int32), np.arange(n, dtype=np.int32),
               diag, rhs, n)
    np.testing.assert_array_equal(x, rhs / diag)
    # the same wrapper on a second structure (plan cache) and back
    first = workloads.configuration("c1")
    second = workloads.configuration("c2", nx=10, ny=9, nz=8)
    for work in (first, second, first):
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(solver, work, expected)
    # same structure, new values: the captured graph is replayed
    for seed in range(3):
        rhs = np.random.default_rng(seed).random(first.n)
        expected = oracle.sptrsv_csc(first.indptr, first.indices, first.data,
                                     rhs, first.n)
        result = solver(first.indptr, first.indices, first.data, rhs, first.n)
        assert relative_error(result, expected) <= TOLERANCE


def test_device_resident_operands(device, oracle):
    work = workloads.configuration("c2", nx=20, ny=20, nz=20)
    expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solver = sptrsv.compile_sptrsv_csc(execution_mode="wavefront",
                                       threads_per_block=128, task_lanes=4)
    operands = [device.to_device(a) for a in
                (work.indptr, work.indices, work.data, work.rhs)]
    call = solver.bind(*operands, work.n)
    for _ in range(3):
        call.launch()
    result = call.result()
    assert relative_error(result, expected) <= TOLERANCE


PLAIN_FIRST_VARIANTS = [
    ("c3", dict(execution_mode="sync_free", threads_per_block=128,
                task_lanes=64, dependence_protocol="pull")),
    ("c2", dict(execution_mode="sync_free", threads_per_block=256,
                task_lanes=4, dependence_protocol="mailbox")),
    ("c2", dict(execution_mode="sync_free", threads_per_block=128,
                task_lanes=4, dependence_protocol="mailbox", tile_rows=None)),
]


@pytest.mark.parametrize("name,options", PLAIN_FIRST_VARIANTS, ids=lambda v: (
    v if isinstance(v, str) else f"{v['dependence_protocol']}-"
    f"{'flat' if 'tile_rows' in v else 'auto'}"))
@pytest.mark.parametrize("grid", [12, 40])
def test_plain_first_polls_see_no_value_of_an_earlier_launch(
        device, oracle, name, options, grid):
    """A poll that accepts a plain load's value must never meet the solution
    of the launch before: one bound call is launched over and over with a new
    right-hand side each time."""
    csr = name == "c3"
    work = (workloads.configuration(name, n=grid ** 3) if csr else
            workloads.configuration(name, nx=grid, ny=grid, nz=grid))
    compile_solver = (sptrsv.compile_sptrsv_csr if csr
                      else sptrsv.compile_sptrsv_csc)
    reference = oracle.sptrsv_csr if csr else oracle.sptrsv_csc
    # (the walkers and the grid sweep poll no value of the solution: the
    # executors that do are what is tested)
    solver = compile_solver(plain_first_polls=True, level_walker=False,
                            band_walker=False, grid_sweep=False, **options)
    operands = [device.to_device(a) for a in
                (work.indptr, work.indices, work.data, work.rhs)]
    call = solver.bind(*operands, work.n)
    assert "lcd_ld_once(&" in solver.hip_lowering.kernel_source
    rng = np.random.default_rng(grid)
    for launch in range(6):
        rhs = work.rhs * (launch + 1) + rng.random(work.n)
        device.copy(operands[3], device.to_device(rhs))
        call.launch()
        call.synchronize()
        expected = reference(work.indptr, work.indices, work.data, rhs, work.n)
        assert relative_error(np.asarray(call.result()), expected) <= TOLERANCE


FULL_SIZE = [("c2", "sptrsv_csc"), ("c4", "ilu0"), ("c3", "sptrsv_csr"),
             ("c5", "sptrsv_csc")]


@pytest.mark.parametrize("name,kind", FULL_SIZE)
def test_full_size_configurations(oracle, name, kind):
    """BASELINE.json's sizes: oracle parity and a size-independent property
    (residual of the solve / L*U == A on the pattern)."""
    print("full size", name, flush=True)
    work = workloads.configuration(name)
    if kind == "ilu0":
        factor = spilu0.compile_ilu0_csr(execution_mode="wavefront",
                                         threads_per_block=128, task_lanes=4,
                                         thread_unroll=1)
        result = factor(work.data.copy(), work.indices, work.indptr)
        expected = oracle.ilu0_csr(work.data, work.indices, work.indptr)
        np.testing.assert_array_equal(result, expected)
        return
    if kind == "sptrsv_csc":
        mode = work.execution_mode
        solver = sptrsv.compile_sptrsv_csc(execution_mode=mode,
                                           threads_per_block=256, task_lanes=4
                                           if name == "c2" else 8)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        from scipy.sparse import csc_matrix as sparse
    else:
        solver = sptrsv.compile_sptrsv_csr(execution_mode="sync_free",
                                           threads_per_block=256, task_lanes=16)
        expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        from scipy.sparse import csr_matrix as sparse
    result = solve_and_check(solver, work, expected)
    matrix = sparse((work.data, work.indices, work.indptr),
                    shape=(work.n, work.n))
    residual = np.asarray(matrix @ result).ravel() - work.rhs
    scale = float(np.max(np.abs(work.rhs)))
    assert float(np.max(np.abs(residual))) <= 1e-10 * max(scale, 1.0) * 10


def test_full_size_headline_defaults(oracle):
    """Configuration 2 on the tiled gathered mailbox and as the decorator
    chooses by itself (the grid sweep; box tiles without it): bit-identical
    to the sequential loop."""
    work = workloads.configuration("c2")
    expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    tuned = sptrsv.compile_sptrsv_csc(
        execution_mode="sync_free", threads_per_block=384, task_lanes=4,
        thread_unroll=1, dependence_protocol="mailbox", tile_rows=4096)
    solve_and_check(tuned, work, expected, exact=True)
    assert tuned.hip_lowering.tile_rows == 4096
    automatic = sptrsv.compile_sptrsv_csc()
    solve_and_check(automatic, work, expected, exact=True)
    plan = automatic.schedule_plan(work.indptr, work.indices, work.data,
                                   work.rhs, work.n)
    assert plan.schedule.execution_mode == "sync_free"
    assert plan.schedule.dependence_protocol == "mailbox"
    assert plan.grid_sweep is not None and plan.grid_sweep[:3] == (128, 128, 128)
    assert automatic.hip_lowering.grid_sweep["workgroups"] == 128
    automatic = sptrsv.compile_sptrsv_csc(grid_sweep=False)
    solve_and_check(automatic, work, expected, exact=True)
    plan = automatic.schedule_plan(work.indptr, work.indices, work.data,
                                   work.rhs, work.n)
    assert plan.schedule.dependence_protocol == "mailbox"
    assert plan.tile_rows == 4096 and automatic.hip_lowering.tile_rows == 4096
    assert 0.6 < plan.dag.tile_locality(4096) < 0.7
    # the power-law matrix keeps no edge inside a tile: flat queue
    work = workloads.configuration("c3", n=100000)
    solver = sptrsv.compile_sptrsv_csr()
    expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solve_and_check(solver, work, expected)
    plan = solver.schedule_plan(work.indptr, work.indices, work.data,
                                work.rhs, work.n)
    assert plan.tile_rows is None and plan.dag.tile_locality(4096) < 0.2


def _bench_settings():
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(
        os.path.abspath(__file__))), "bench.py")
    spec = importlib.util.spec_from_file_location("lcd_bench", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module.TUNED


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_full_size_under_bench_settings(oracle, name):
    """Every BASELINE configuration at full size with exactly the executor
    settings bench.py times (its TUNED table, imported, not retyped).  ILU0
    and the mailbox SpTRSV must be bit-identical to the sequential loop; the
    lane-strided CSR pull meets the element-wise bound."""
    options = dict(_bench_settings()[name])
    print("full size, bench settings", name, options, flush=True)
    work = workloads.configuration(name)
    if work.kind == "ilu0_csr":
        factor = spilu0.compile_ilu0_csr(**options)
        result = factor(work.data.copy(), work.indices, work.indptr)
        expected = oracle.ilu0_csr(work.data, work.indices, work.indptr)
        np.testing.assert_array_equal(result, expected)
        assert factor.hip_lowering.published_array == "A_data"
        return
    if work.kind == "sptrsv_csc":
        solver = sptrsv.compile_sptrsv_csc(**options)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(solver, work, expected, exact=True)
        if name in ("c1", "c5"):
            # the chain runs on the band walker, the small grid on the level
            # walker, each with its own workgroup
            assert (solver.hip_lowering.band_walker if name == "c5"
                    else solver.hip_lowering.level_walker)
            assert solver.hip_lowering.tile_rows is None
            assert solver.current_schedule.threads_per_block == 1024
            return
        # the grid of configuration 2 runs on the grid sweep, whose workgroup
        # is its bundles' and helpers' wavefronts
        assert solver.hip_lowering.grid_sweep is not None
        assert solver.hip_lowering.tile_rows is None
        assert solver.current_schedule.threads_per_block == (
            solver.hip_lowering.grid_sweep["threads"])
        return
    else:
        solver = sptrsv.compile_sptrsv_csr(**options)
        expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        solve_and_check(solver, work, expected)
    assert solver.hip_lowering.task_lanes == options["task_lanes"]
    assert solver.current_schedule.threads_per_block == (
        options["threads_per_block"])


@pytest.mark.parametrize("options", [
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4,
         dependence_protocol="push"),
    dict(execution_mode="sync_free", threads_per_block=128, task_lanes=4,
         dependence_protocol="counter"),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=4,
         dependence_protocol="mailbox", gather_messages=False),
    dict(execution_mode="sync_free", threads_per_block=256, task_lanes=4,
         dependence_protocol="mailbox", tile_rows=512),
], ids=["push", "counter", "mailbox-slots", "mailbox-tiled"])
@pytest.mark.parametrize("switch", ["full_fences", "dynamic_fetch"])
def test_conservative_builds_are_the_control(oracle, options, switch):
    """The same executors compiled with the HIP memory model's agent-scope
    release/acquire fences (``full_fences``) instead of the
    wait-for-completion scheme, and with task batches handed out by the
    global counter (``dynamic_fetch``) instead of round-robin: same results
    to the same bar."""
    print("control build", switch, options, flush=True)
    work = workloads.configuration("c2", nx=40, ny=36, nz=20)
    expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    solver = sptrsv.compile_sptrsv_csc(**options, **{switch: True})
    exact = options["dependence_protocol"] == "mailbox"
    solve_and_check(solver, work, expected, exact=exact)
    macro = {"full_fences": "#define LCD_FULL_FENCES 1",
             "dynamic_fetch": "#define LCD_DYNAMIC_FETCH 1"}[switch]
    assert macro in solver.hip_lowering.source


def test_conservative_builds_csr_and_ilu0(oracle):
    work = workloads.configuration("c3", n=40000)
    expected = oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                 work.rhs, work.n)
    for extra in (dict(full_fences=True), dict(dynamic_fetch=True),
                  dict(full_fences=True, value_flags=False)):
        print("control build csr", extra, flush=True)
        solver = sptrsv.compile_sptrsv_csr(
            execution_mode="sync_free", threads_per_block=128, task_lanes=16,
            dependence_protocol="pull", **extra)
        solve_and_check(solver, work, expected)
    work = workloads.configuration("c4", nx=64, ny=48)
    expected = oracle.ilu0_csr(work.data, work.indices, work.indptr)
    for extra in (dict(full_fences=True), dict(dynamic_fetch=True)):
        print("control build ilu0", extra, flush=True)
        factor = spilu0.compile_ilu0_csr(
            execution_mode="sync_free", threads_per_block=128, task_lanes=64,
            thread_unroll=1, dependence_protocol="pull", **extra)
        result = factor(work.data.copy(), work.indices, work.indptr)
        np.testing.assert_array_equal(result, expected)


def test_plain_kernel_on_an_edge_free_matrix(oracle):
    """The executor-free kernel (one task group per iteration, no dependence
    protocol: compiler/cuda_lowering.py:519-532, launcher :673-735) run on the
    GPU.  The README loop on a diagonal matrix has no edges, so running every
    column at once is legal; with edges present the same kernel would race,
    which is why the decorator never selects it."""
    from lcd_amd import hip_runtime
    from lcd_amd.dependence import analyze_dependences
    from lcd_amd.hip_lowering import lower_to_hip
    module = ast.parse(inspect.getsource(sptrsv.sptrsv_csc_loop))
    props = sptrsv.FUNCTION_PROPS_CSC
    analysis = analyze_dependences(module, "i", props)
    rng = np.random.default_rng(5)
    n = 100_003
    indptr = np.arange(n + 1, dtype=np.int32)
    indices = np.arange(n, dtype=np.int32)
    data = rng.uniform(1.0, 2.0, n)
    rhs = rng.standard_normal(n)
    expected = oracle.sptrsv_csc(indptr, indices, data, rhs, n)
    np.testing.assert_array_equal(expected, rhs / data)
    for extra in (dict(), dict(thread_loop_iterator="j", task_lanes=4)):
        print("plain kernel", extra, flush=True)
        lowering = lower_to_hip(
            module, "i", reductions=analysis, function_props=props,
            execution_mode="plain", wavefront_threads_per_block=128, **extra)
        assert lowering.auxiliary_arguments == []
        compiled = hip_runtime.compile_hip_module(lowering, {"np": np})
        arguments = {"Ap": indptr, "Ai": indices, "Ax": data, "b": rhs, "n": n}
        prepared = hip_runtime.prepare_hip_arguments(lowering, arguments, None,
                                                     {"np": np})
        result = hip_runtime.execute_hip_call(compiled, lowering, prepared,
                                              {"np": np})
        np.testing.assert_array_equal(result, expected)


def _smooth(x, w, n):
    for i in range(n):
        x[i] = x[i] + w[i] * x[(i * 7) % n]
    return x


@pytest.mark.parametrize("mode", ["sync_free", "wavefront"])
def test_unrecognised_dependence_runs_in_sequential_order(mode):
    """A loop whose dependence no edge rule enumerates is kept as the
    complete order (chain i -> i + 1): the decorated function runs, one
    iteration after the other, and equals the undecorated loop bit for bit."""
    import warnings

    from lcd_amd import parallel
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        solver = parallel(loop="i", execution_mode=mode)(_smooth)
    assert any("complete order" in str(w.message) for w in caught)
    rng = np.random.default_rng(3)
    n = 700
    x0, w = rng.standard_normal(n), rng.uniform(-0.5, 0.5, n)
    print("conservative", mode, n, flush=True)
    expected = _smooth(x0.copy(), w, n)
    result = solver(x0.copy(), w, n)
    np.testing.assert_array_equal(result, expected)
    successors, _ = solver.build_dag(x0, w, n)
    assert successors == [[k + 1] for k in range(n - 1)] + [[]]


def _random_lower_triangle(rng, kind, n):
    """Strictly lower part scaled by 0.1 plus a diagonal in [1, 2): random
    sparsity, a band, a 5-point grid, or an arrow (first column and last row
    full: one task with n - 1 consumers, one with n - 1 producers)."""
    import scipy.sparse as sp
    if kind == "random":
        per_row = float(rng.choice([0.5, 2, 6, 20]))
        lower = sp.random(n, n, density=min(1.0, per_row / n),
                          random_state=int(rng.integers(1 << 30)),
                          format="csr")
    elif kind == "band":
        width = min(int(rng.integers(1, 12)), n - 1)
        lower = sp.csr_matrix((n, n)) if width < 1 else sp.diags(
            [rng.uniform(-1, 1, n)] * width,
            [-k for k in range(1, width + 1)], shape=(n, n), format="csr")
    elif kind == "grid":
        side = max(1, int(np.sqrt(n)))
        n = side * side
        shift = sp.diags([np.ones(side)], [-1], shape=(side, side))
        lower = (sp.kron(sp.identity(side), shift)
                 + sp.kron(shift, sp.identity(side))).tocsr()
    else:
        lower = sp.lil_matrix((n, n))
        lower[:, 0] = 1.0
        lower[n - 1, :] = 1.0
        lower = lower.tocsr()
    return sp.tril(lower, -1) * 0.1 + sp.diags(rng.uniform(1, 2, n)), n


@pytest.mark.parametrize("seed", [3, 4])
def test_random_structures_under_random_schedules(oracle, seed):
    """Random matrices (sizes 1 to 20 000 around the wavefront size and the
    tile sizes) solved under randomly drawn executors, protocols, lanes per
    task, tile sizes, grid caps and fetch variants, each against the oracle;
    ILU0 of the symmetrised pattern bit-identical to the sequential loop."""
    import scipy.sparse as sp
    rng = np.random.default_rng(seed)
    for trial in range(8):
        n = int(rng.choice([1, 2, 63, 65, 300, 1000, 5000, 20000]))
        kind = str(rng.choice(["random", "band", "grid", "arrow"]))
        lower, n = _random_lower_triangle(rng, kind, n)
        rhs = rng.standard_normal(n)
        options = dict(
            execution_mode=str(rng.choice(["sync_free", "wavefront"])),
            threads_per_block=int(rng.choice([64, 128, 192, 256, 384])),
            task_lanes=int(rng.choice([1, 2, 4, 8, 16, 64])))
        persistent = options["execution_mode"] == "sync_free"
        if persistent:
            options["tile_rows"] = [None, 32, 64, 500, 4096][
                int(rng.integers(5))]
            options["resident_waves_per_cu"] = [None, 1, 0.25][
                int(rng.integers(3))]
            options["pipeline_fetch"] = bool(rng.integers(2))
        print("random structure", seed, trial, kind, n, options, flush=True)
        for storage, tiled, protocols in (
                ("csc", "mailbox", ["mailbox", "push", "counter"]),
                ("csr", "pull", ["pull", "counter"])):
            matrix = (sp.csc_matrix(lower) if storage == "csc"
                      else sp.csr_matrix(lower))
            matrix.sort_indices()
            indptr = matrix.indptr.astype(np.int32)
            indices = matrix.indices.astype(np.int32)
            solve = getattr(oracle, f"sptrsv_{storage}")
            expected = solve(indptr, indices, matrix.data, rhs, n)
            compile_solver = getattr(sptrsv, f"compile_sptrsv_{storage}")
            for protocol in protocols if persistent else ["counter"]:
                chosen = dict(options, dependence_protocol=protocol)
                if protocol != tiled:
                    chosen.pop("tile_rows", None)
                result = compile_solver(**chosen)(
                    indptr, indices, matrix.data, rhs, n)
                assert relative_error(result, expected) <= TOLERANCE, (
                    trial, storage, chosen)
        if kind == "arrow":
            continue
        pattern = sp.csr_matrix(lower + lower.T * 0.5)
        pattern.sort_indices()
        indptr = pattern.indptr.astype(np.int32)
        indices = pattern.indices.astype(np.int32)
        expected = oracle.ilu0_csr(pattern.data.copy(), indices, indptr)
        chosen = dict(execution_mode=options["execution_mode"],
                      threads_per_block=int(rng.choice([64, 128, 256])))
        if persistent:
            chosen.update(task_lanes=int(rng.choice([8, 64])),
                          dependence_protocol="pull",
                          publish_values=bool(rng.integers(2)),
                          look_ahead=bool(rng.integers(2)))
        result = spilu0.compile_ilu0_csr(**chosen)(
            pattern.data.copy(), indices, indptr)
        np.testing.assert_array_equal(result, expected)

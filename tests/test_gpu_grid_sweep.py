"""The grid sweep on the GPU (lcd_amd/hip_grid_sweep.py): the solve of an
axis stencil on a three-dimensional grid with a lane per grid line, against
the sequential loop of the oracle, bit for bit.  Every call goes through the
decorator and the C ABI underneath it."""

import numpy as np
import pytest

from lcd_amd import hip_runtime, workloads
from lcd_amd.demo import sptrsv

pytestmark = pytest.mark.gpu

SWEEP = dict(execution_mode="sync_free", task_lanes=4, thread_unroll=1,
             dependence_protocol="mailbox", grid_sweep=True)


def random_values(work, seed):
    """The stencil's structure with values that differ entry by entry, so
    that a coefficient taken from the wrong direction or the wrong node
    shows."""
    rng = np.random.default_rng(seed)
    values = work.data.copy()
    off = values < 0
    values[off] = -1.0 + rng.uniform(-0.3, 0.3, int(off.sum()))
    values[~off] = 6.0 + rng.uniform(-0.5, 0.5, int((~off).sum()))
    return values


def grid(shape):
    return workloads.configuration("c2", nx=shape[0], ny=shape[1], nz=shape[2])


@pytest.mark.parametrize("shape", [(24, 20, 12), (40, 20, 28), (33, 17, 9),
                                   (16, 16, 70), (5, 3, 2)])
@pytest.mark.parametrize("sweep_shape", [(8, 1, 2, 1), (16, 1, 2, 2),
                                         (8, 2, 2, 1), (16, 1, 1, 1),
                                         (8, 2, 1, 2)])
def test_grid_sweep_is_the_sequential_loop(oracle, shape, sweep_shape):
    """Grids that the bundles of 8 x 8 and 16 x 4 lines divide and grids
    they do not, one to four bundles per workgroup, one and two steps
    between the z rows: the same bits as the sequential loop."""
    print("grid sweep", shape, sweep_shape, flush=True)
    work = grid(shape)
    values = random_values(work, 7)
    expected = oracle.sptrsv_csc(work.indptr, work.indices, values, work.rhs,
                                 work.n)
    solver = sptrsv.compile_sptrsv_csc(sweep_shape=sweep_shape, **SWEEP)
    result = solver(work.indptr, work.indices, values, work.rhs, work.n)
    plan = solver.schedule_plan(work.indptr, work.indices, values, work.rhs,
                                work.n)
    assert plan.grid_sweep == tuple(shape) + tuple(sweep_shape)
    assert solver.hip_lowering.grid_sweep["nx"] == shape[0]
    np.testing.assert_array_equal(result, expected)


def test_row_form_of_the_same_solve(oracle):
    """The pull-shaped loop (CSR: ``x[i] = b[i]; for j in row: x[i] -= Ax[j] *
    x[Ai[j]]; x[i] /= d``) over the same grid runs on the same sweep: the row
    is the incoming listing, the element's first value is staged with the
    node loads.  Bit-identical to its own sequential loop."""
    from scipy.sparse import csc_matrix
    work = grid((36, 20, 12))
    values = random_values(work, 5)
    rows = csc_matrix((values, work.indices, work.indptr),
                      shape=(work.n, work.n)).tocsr()
    rows.sort_indices()                     # the diagonal ends every row
    indptr = rows.indptr.astype(np.int32)
    indices = rows.indices.astype(np.int32)
    expected = oracle.sptrsv_csr(indptr, indices, rows.data, work.rhs, work.n)
    solver = sptrsv.compile_sptrsv_csr(
        execution_mode="sync_free", task_lanes=4, thread_unroll=1,
        dependence_protocol="pull", grid_sweep=True)
    result = solver(indptr, indices, rows.data, work.rhs, work.n)
    assert solver.hip_lowering.grid_sweep is not None
    np.testing.assert_array_equal(result, expected)


def test_matrix_values_and_right_hand_side_are_picked_up(device, oracle):
    """The decorated function called again with other matrix values (the
    records are laid out again: their digest has changed) and another
    right-hand side (staged in front of every solve); a bound call whose
    matrix array changes in place needs ``update_values()``, its right-hand
    side is read at every launch."""
    work = grid((40, 24, 20))
    solver = sptrsv.compile_sptrsv_csc(**SWEEP)
    for seed in (1, 2, 3):
        values = random_values(work, seed)
        rhs = np.random.default_rng(seed + 10).standard_normal(work.n)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, values, rhs,
                                     work.n)
        np.testing.assert_array_equal(
            solver(work.indptr, work.indices, values, rhs, work.n), expected)
    values = random_values(work, 4)
    operands = [device.to_device(a) for a in
                (work.indptr, work.indices, values, work.rhs)]
    call = solver.bind(*operands, work.n)
    for launch in range(3):
        rhs = np.random.default_rng(launch).random(work.n)
        device.copy(operands[3], device.to_device(rhs))
        call.launch()
        np.testing.assert_array_equal(
            call.result(), oracle.sptrsv_csc(work.indptr, work.indices, values,
                                             rhs, work.n))
    changed = random_values(work, 5)
    device.copy(operands[2], device.to_device(changed))
    call.update_values()
    call.launch()
    np.testing.assert_array_equal(
        call.result(), oracle.sptrsv_csc(work.indptr, work.indices, changed,
                                         rhs, work.n))


def test_divisions_the_prepared_reciprocal_does_not_serve(oracle):
    """Tiny, huge and denormal divisors and numerators, a zero right-hand
    side, an infinite entry: the checked division of a step divides again in
    full where the prepared reciprocal is not the division, and the bits are
    the sequential loop's."""
    work = grid((24, 16, 8))
    values = random_values(work, 9)
    diagonal = work.indptr[:-1]
    rng = np.random.default_rng(0)
    picks = rng.choice(work.n, 40, replace=False)
    specials = [1e-200, 1e250, 5e-324, 1e-310, 3.0, 1e100, 1e-100, -2.5e-300]
    for k, node in enumerate(picks):
        values[diagonal[node]] = specials[k % len(specials)]
    rhs = work.rhs.copy()
    rhs[picks[:10]] = 0.0
    rhs[picks[10:14]] = [1e-305, 1e300, -1e-320, np.inf]
    solver = sptrsv.compile_sptrsv_csc(**SWEEP)
    with np.errstate(all="ignore"):
        expected = oracle.sptrsv_csc(work.indptr, work.indices, values, rhs,
                                     work.n)
    result = solver(work.indptr, work.indices, values, rhs, work.n)
    np.testing.assert_array_equal(result, expected)
    zero = solver(work.indptr, work.indices, random_values(work, 2),
                  np.zeros(work.n), work.n)
    assert not np.any(zero) and not np.any(np.signbit(zero))


def test_the_scheduler_takes_the_sweep_for_grids_only(oracle):
    """By itself the decorator runs a three-dimensional grid beyond the
    level walker's size on the sweep; a small grid, a two-dimensional grid
    and a matrix that is no grid keep their executors, and asking for the
    sweep on one of those is an error."""
    solver = sptrsv.compile_sptrsv_csc()
    for shape, swept in (((32, 24, 16), True), ((12, 12, 12), False)):
        work = grid(shape)
        expected = oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
        result = solver(work.indptr, work.indices, work.data, work.rhs, work.n)
        np.testing.assert_array_equal(result, expected)
        plan = solver.schedule_plan(work.indptr, work.indices, work.data,
                                    work.rhs, work.n)
        assert (plan.grid_sweep is not None) == swept, shape
    flat = workloads.configuration("c1", nx=96, ny=96)
    plan = solver.schedule_plan(flat.indptr, flat.indices, flat.data, flat.rhs,
                                flat.n)
    assert plan.grid_sweep is None
    band = workloads.configuration("c5", n=20000)
    forced = sptrsv.compile_sptrsv_csc(**SWEEP)
    with pytest.raises(ValueError, match="grid_sweep=True"):
        forced(band.indptr, band.indices, band.data, band.rhs, band.n)


def test_an_abandoned_launch_leaves_the_sweep_usable(device, oracle):
    """A wait that cannot end -- forced from the host: the counter the
    workgroups take their places from starts at one, so no workgroup takes
    place 0 and the faces it would have sent never come -- ends through the
    kernels' own bounded waits, the call raises, and the same bound call
    solves correctly afterwards (faces and counters are put back)."""
    work = grid((32, 24, 16))
    values = random_values(work, 3)
    solver = sptrsv.compile_sptrsv_csc(spin_limit=20000, **SWEEP)
    operands = [device.to_device(a) for a in
                (work.indptr, work.indices, values, work.rhs)]
    call = solver.bind(*operands, work.n)
    call.launch()
    expected = oracle.sptrsv_csc(work.indptr, work.indices, values, work.rhs,
                                 work.n)
    np.testing.assert_array_equal(call.result(), expected)
    claim = call.device_value("_lcd_sw_claim")
    device.copy(claim, device.to_device(np.array([1, 0, 0, 0], np.int32)))
    call.launch()
    with pytest.raises(hip_runtime.ExecutorWatchdogError):
        call.synchronize()
    call.launch()
    np.testing.assert_array_equal(call.result(), expected)

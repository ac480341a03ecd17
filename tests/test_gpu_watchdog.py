"""Failure handling of the persistent executor on the GPU: a wait that can
never be satisfied ends through the kernel's own bounded spin (every
wavefront exits normally), the host raises ExecutorWatchdogError, and the
same plan runs correctly afterwards.

The condition is forced from the host: in the task queue handed to the
executor the entry of node 0 is overwritten with a second copy of the last
node (a sink: nothing depends on it), so whatever node 0 would have produced
(a counter decrement, a message, a done flag, a final value) never comes.
All array sizes stay as they are."""

import ast
import inspect
from dataclasses import replace

import numpy as np
import pytest

from lcd_amd import dag_preprocessing as P
from lcd_amd import hip_runtime, workloads
from lcd_amd.dag_codegen import create_dag_plan, direct_dependence
from lcd_amd.demo import sptrsv
from lcd_amd.dependence import analyze_dependences
from lcd_amd.hip_lowering import lower_to_hip

pytestmark = pytest.mark.gpu

CASES = [
    ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC, "counter", {}),
    ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC, "push", {}),
    ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC, "mailbox",
     dict(gather_messages=False)),
    ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC, "mailbox", {}),
    ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC, "mailbox",
     dict(task_records=False)),
    ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC, "mailbox",
     dict(tile_rows=512)),
    ("sptrsv_csr_loop", sptrsv.FUNCTION_PROPS_CSR, "pull", {}),
    ("sptrsv_csr_loop", sptrsv.FUNCTION_PROPS_CSR, "pull",
     dict(value_flags=False)),
    ("sptrsv_csr_loop", sptrsv.FUNCTION_PROPS_CSR, "pull",
     dict(tile_rows=512)),
]


@pytest.mark.parametrize(
    "name,props,protocol,extra", CASES,
    ids=["counter", "push", "mailbox-slots", "mailbox-gathered",
         "mailbox-staged", "mailbox-tiled", "pull-values", "pull-flags", "pull-tiled"])
def test_unsatisfiable_wait_trips_the_watchdog(oracle, name, props, protocol,
                                               extra):
    _trip_and_recover(oracle, name, props, protocol, extra,
                      dict(spin_limit=3000))


@pytest.mark.parametrize("protocol,extra", [
    ("counter", {}), ("mailbox", dict(tile_rows=512)), ("pull", {})])
def test_default_watchdog_gives_up_within_seconds(oracle, protocol, extra):
    """Without a caller-chosen spin limit the plan's own limit (scaled to
    the 127 levels of this DAG) applies: the stuck launch ends in seconds,
    not in the twenty-odd the fixed default took."""
    import time
    name, props = (("sptrsv_csr_loop", sptrsv.FUNCTION_PROPS_CSR)
                   if protocol == "pull"
                   else ("sptrsv_csc_loop", sptrsv.FUNCTION_PROPS_CSC))
    start = time.perf_counter()
    _trip_and_recover(oracle, name, props, protocol, extra, {})
    elapsed = time.perf_counter() - start
    print(f"default watchdog {protocol}: {elapsed:.2f} s", flush=True)
    assert elapsed < 10.0


def _trip_and_recover(oracle, name, props, protocol, extra, limit):
    print("watchdog", name, protocol, extra, limit, flush=True)
    function = getattr(sptrsv, name)
    module = ast.parse(inspect.getsource(function))
    analysis = analyze_dependences(module, "i", props)
    plan = create_dag_plan(analysis.ordering_dependences, None, "i",
                           ["Ap", "Ai", "Ax", "b", "n"])
    lowering = lower_to_hip(
        module, "i", reductions=analysis, function_props=props,
        execution_mode="sync_free", thread_loop_iterator="j", task_lanes=4,
        wavefront_threads_per_block=64, dependence_protocol=protocol,
        direct_dependence=(None if protocol == "counter"
                           else direct_dependence(plan, "j")),
        **limit, **extra)
    assert lowering.dependence_protocol == protocol
    compiled = hip_runtime.compile_hip_module(lowering, {"np": np})

    csc = name == "sptrsv_csc_loop"
    work = workloads.configuration("c1")
    if csc:
        indptr, indices, data = work.indptr, work.indices, work.data
        expected = oracle.sptrsv_csc(indptr, indices, data, work.rhs, work.n)
        rule = oracle.rule_sptrsv_csc(indptr, indices)
    else:
        import scipy.sparse as sp
        matrix = sp.csc_matrix((work.data, work.indices, work.indptr),
                               shape=(work.n, work.n)).tocsr()
        matrix.sort_indices()
        indptr = matrix.indptr.astype(np.int32)
        indices = matrix.indices.astype(np.int32)
        data = matrix.data
        expected = oracle.sptrsv_csr(indptr, indices, data, work.rhs, work.n)
        rule = oracle.rule_sptrsv_csr(indptr, indices)
    device = hip_runtime.default_device()
    dag = device.dag_build([rule], work.n, levels=True,
                           incoming=protocol == "mailbox")
    good = P.execution_data_from_device_dag(
        dag, "sync_free", True, pushed=protocol == "push",
        mailbox=protocol == "mailbox", tile_rows=lowering.tile_rows,
        record_lanes=lowering.task_record_lanes)
    assert lowering.tile_rows == extra.get("tile_rows")
    # node 0 (level 0) never runs; the last node of the last level runs twice
    order = "tile_nodes" if lowering.tile_rows else "wavefronts"
    nodes = dag.host(order).copy()
    assert nodes[0] == 0 and dag.host("dag_ptr")[nodes[-1] + 1] == (
        dag.host("dag_ptr")[nodes[-1]])       # (a sink: no successors)
    nodes[0] = nodes[-1]
    bad = replace(good, task_nodes=device.to_device(nodes))
    arguments = {"Ap": indptr, "Ai": indices, "Ax": data, "b": work.rhs,
                 "n": work.n}
    prepared = hip_runtime.prepare_hip_arguments(lowering, arguments, bad,
                                                 {"np": np})
    with pytest.raises(hip_runtime.ExecutorWatchdogError):
        hip_runtime.execute_hip_call(compiled, lowering, prepared, {"np": np})
    # the status word is re-armed: the intact queue solves the system
    prepared = hip_runtime.prepare_hip_arguments(lowering, arguments, good,
                                                 {"np": np})
    result = hip_runtime.execute_hip_call(compiled, lowering, prepared,
                                          {"np": np})
    scale = float(np.max(np.abs(expected)))
    assert float(np.max(np.abs(result - expected))) / scale <= 1e-12


@pytest.mark.parametrize("lanes,tpb", [(8, 64), (64, 128)],
                         ids=["done-flags", "published-values"])
def test_ilu0_pivot_wait_trips_the_watchdog(oracle, lanes, tpb):
    """The per-pivot wait of ILU0 (pull on the task's own loop; polls of the
    producers' published values with one row per wavefront): a producer that
    never runs ends the launch through the watchdog, and the next call with
    the intact queue factorises."""
    from lcd_amd.demo import spilu0
    from lcd_amd.structural_lookups import (create_structural_lookup_plan,
                                            materialize_structural_lookups)
    print("watchdog ilu0 pull", lanes, flush=True)
    module = ast.parse(inspect.getsource(spilu0.ilu0_csr))
    props = spilu0.FUNCTION_PROPS
    analysis = analyze_dependences(module, "i", props)
    plan = create_dag_plan(analysis.ordering_dependences, None, "i",
                           ["A_data", "A_indices", "A_indptr", "n"])
    lookups = create_structural_lookup_plan(module, props)
    lowering = lower_to_hip(
        module, "i", reductions=analysis, function_props=props,
        execution_mode="sync_free", thread_loop_iterator="j_ptr",
        task_lanes=lanes, wavefront_threads_per_block=tpb,
        dependence_protocol="pull",
        direct_dependence=direct_dependence(plan, "j_ptr"),
        structural_lookups=lookups, spin_limit=3000)
    assert lowering.dependence_protocol == "pull"
    assert "_lcd_blocked" in lowering.kernel_source
    assert (lowering.published_array == "A_data") == (lanes == 64)
    compiled = hip_runtime.compile_hip_module(lowering, {"np": np})
    work = workloads.configuration("c4", nx=40, ny=30)
    device = hip_runtime.default_device()
    dag = device.dag_build(
        [oracle.rule_ilu0_csr(work.indptr, work.indices)], work.n, levels=True)
    good = P.execution_data_from_device_dag(dag, "sync_free", True)
    nodes = dag.host("wavefronts").copy()
    assert nodes[0] == 0
    nodes[0] = nodes[-1]
    bad = replace(good, task_nodes=device.to_device(nodes))
    arguments = {"A_data": work.data.copy(), "A_indices": work.indices,
                 "A_indptr": work.indptr}
    tables = materialize_structural_lookups(lookups, arguments, device)
    prepared = hip_runtime.prepare_hip_arguments(
        lowering, arguments, P.attach_auxiliary_values(bad, tables),
        {"np": np})
    with pytest.raises(hip_runtime.ExecutorWatchdogError):
        hip_runtime.execute_hip_call(compiled, lowering, prepared, {"np": np})
    arguments["A_data"] = work.data.copy()
    prepared = hip_runtime.prepare_hip_arguments(
        lowering, arguments, P.attach_auxiliary_values(good, tables),
        {"np": np})
    result = hip_runtime.execute_hip_call(compiled, lowering, prepared,
                                          {"np": np})
    np.testing.assert_array_equal(
        result, oracle.ilu0_csr(work.data, work.indices, work.indptr))

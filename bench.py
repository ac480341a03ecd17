#!/usr/bin/env python3
"""Benchmark of the `@parallel` solve path on one MI355X.

A step is one solve (SpTRSV) or one factorisation (ILU0) of a synthetic
configuration whose operands are already resident in HBM: the lifted output
is cleared on the device, the executor state is reset, and the generated
kernels run (all replayed from one hipGraph).  Host/device copies, the DAG
inspection and hiprtc compilation happen before the timed region and are
reported separately.

Headline workload (``value``, ``ms_per_step``, ``roofline``,
``cpu_baseline``): configuration 2 of BASELINE.json (SpTRSV-CSC on the lower
factor of the 3-D 7-point Laplacian, 128^3).  Without ``--config`` the same
JSON line also carries, under ``configs``, one record for each of the five
configurations and for configuration 2 under the level-launched (wavefront)
executor: solve time, GFLOP/s, GB/s, roofline fraction of the dominant kernel
with its measured traffic, the dependency-latency bound ``levels x hand-off``,
the single-core CPU baseline and the error against the sequential loop, the
way the reference's harness reports per matrix
(benchmark/sptrsv_benchmark.py:420-431,626, benchmark/spilu0_benchmark.py:767).
Prints ONE JSON line.
"""

import argparse
import gc
import json
import os
import sys
import threading
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0
METRIC = "SpTRSV/SpILU0 solve ms, GFLOP/s, HBM GB/s (% roofline) on 1 MI355X"


# Executor settings per configuration (the fastest measured on MI355X; every
# one can be overridden on the command line).
TUNED = {
    # (a small DAG with narrow levels: the level walker, one wavefront that
    # takes a level per step, chosen per plan; --level-walker 0 gives the tiles
    # of 1024 rows with 256 threads)
    "c1": dict(execution_mode="sync_free", task_lanes=4,
               thread_unroll=1, dependence_protocol="mailbox", spin_sleep=0),
    # (an axis stencil on a grid: the grid sweep, chosen per plan -- a lane per
    # grid line, a wavefront per bundle of 8 x 8 lines; --grid-sweep 0 gives
    # the box tiles of 128 x 8 x 4 points with 512 threads)
    "c2": dict(execution_mode="sync_free", task_lanes=4, thread_unroll=1,
               dependence_protocol="mailbox", spin_sleep=0),
    "c3": dict(execution_mode="sync_free", threads_per_block=128,
               task_lanes=64, thread_unroll=1,
               dependence_protocol="pull", tile_rows=None),
    # (rows of nine entries: the row lives in registers and the searches of
    # the pivot loop come from the inspector's tables, both chosen per plan)
    "c4": dict(execution_mode="sync_free", threads_per_block=640,
               task_lanes=64, thread_unroll=1, dependence_protocol="pull",
               tile_rows=1024, tile_positions=9216),
    # (a chain: the band walker, one wavefront in program order, chosen per
    # plan; --band-walker 0 gives the tiles of 8192 rows with 128 threads)
    "c5": dict(execution_mode="sync_free", task_lanes=8,
               thread_unroll=1, dependence_protocol="mailbox", spin_sleep=0),
}


# HBM bytes per launch of the dominant kernel, from rocprofv3 --pmc FETCH_SIZE /
# WRITE_SIZE runs scaled by the copy-probe kernel: profiles/traffic.json holds
# one entry per profiled (configuration, executor settings) next to the
# summary it was taken from; anything not profiled reports null.
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")
OVERRIDE_VARIABLES = ("LCD_HIP_OVERRIDE_DIR", "LCD_HIP_EXTRA_OPTIONS")
# Steps of the sub-records (the headline uses --steps / --warmup): the chain
# of configuration 5 takes long per solve.
# Under level launches (--mode wavefront): a task per lane whose record of
# four incoming entries comes in with vector loads, read from operands laid
# out in level order (128^3 grid: 1.00 ms with 128 threads per block, 0.98 with
# 64; four lanes per task 1.11 ms).
# ILU0: a row per wavefront, the row in registers and the pivot loop's
# searches in tables as in the persistent executor, plain loads (9-point
# 1024^2: 16.6 ms; four lanes per row with searches 27.8 ms).
TUNED_LEVEL_LAUNCHES = {
    "c2": dict(task_lanes=1, threads_per_block=64),
    "c4": dict(task_lanes=64, threads_per_block=128,
               dependence_protocol="pull"),
}

SUB_STEPS = {"c1": (50, 10), "c2": (50, 10), "c3": (50, 10), "c4": (20, 3),
             "c5": (3, 1)}
CPU_SECONDS_SUB = 3.0
RTOL, ATOL_SCALE = 1e-12, 1e-15


def traffic_key(config, mode, protocol, lanes, tile_rows, tile_box=None,
                walker=False):
    key = f"{config}|{mode}|{protocol}|lanes={lanes}|tile_rows={tile_rows or 0}"
    if walker:
        key = f"{config}|{mode}|{protocol}|{walker}"
    if tile_box:
        key += "|box=" + "x".join(str(extent) for extent in tile_box)
    return key


def measured_traffic(key):
    try:
        with open(TRAFFIC_FILE) as handle:
            entry = json.load(handle).get(key)
    except (OSError, ValueError):
        return None
    return None if entry is None else int(entry["bytes_per_launch"])


def elementwise_error(got, expected):
    """max_i |got_i - ref_i| / (|ref_i| + 1e-3 max|ref|): at most 1e-12 exactly
    when |got - ref| <= 1e-12 |ref| + 1e-15 max|ref| holds for every element
    (the reference's own check is element-wise with rtol 1e-10 / atol 1e-12,
    compiler/e2e_tests/test_sptrsv_e2e.py:64-69; this one is tighter)."""
    floor = float(np.max(np.abs(expected))) * ATOL_SCALE / RTOL
    return float(np.max(np.abs(got - expected) / (np.abs(expected) + floor)))


def hip_runtime_module():
    from lcd_amd import hip_runtime
    return hip_runtime


def build_solver(work, args, config):
    from lcd_amd.demo import spilu0, sptrsv
    options = {} if args.auto else dict(TUNED[config])
    if args.mode:
        options["execution_mode"] = args.mode
        if args.mode != TUNED[config]["execution_mode"] and not args.auto:
            options.pop("tile_rows", None)
            options.pop("spin_sleep", None)
            options.pop("resident_waves_per_cu", None)
            options.pop("dependence_protocol", None)
            if args.mode == "wavefront":
                options.update(TUNED_LEVEL_LAUNCHES.get(config, {}))
    if args.tpb:
        options["threads_per_block"] = args.tpb
    if args.lanes:
        options["task_lanes"] = args.lanes
    if args.unroll:
        options["thread_unroll"] = args.unroll
    if args.protocol:
        options["dependence_protocol"] = args.protocol
    if args.waves_per_cu:
        options["resident_waves_per_cu"] = args.waves_per_cu
    if args.spin_sleep is not None:
        options["spin_sleep"] = args.spin_sleep
    if args.tile_rows is not None:
        options["tile_rows"] = args.tile_rows or None
    if args.tile_positions:
        options["tile_positions"] = args.tile_positions
    if args.tile_box:
        options["tile_box"] = (
            None if args.tile_box == "none" else "auto"
            if args.tile_box == "auto"
            else tuple(int(extent) for extent in args.tile_box.split("x")))
    if args.segment_capacity:
        options["segment_capacity"] = args.segment_capacity
    if args.level_gather:
        options["level_gather"] = True
    if args.band_walker is not None:
        options["band_walker"] = bool(args.band_walker)
        if not args.band_walker and config == "c5" and not args.auto:
            options.setdefault("threads_per_block", 128)
            options.setdefault("tile_rows", 8192)
    if args.grid_sweep is not None:
        options["grid_sweep"] = bool(args.grid_sweep)
        if not args.grid_sweep and config == "c2" and not args.auto:
            options.setdefault("threads_per_block", 512)
            options.setdefault("tile_rows", 4096)
    if args.sweep_shape:
        options["sweep_shape"] = tuple(
            int(extent) for extent in args.sweep_shape.split(","))
    if args.level_walker is not None:
        options["level_walker"] = bool(args.level_walker)
        if not args.level_walker and config == "c1" and not args.auto:
            options.setdefault("threads_per_block", 256)
            options.setdefault("tile_rows", 1024)
    if args.no_queue_loads:
        options["queue_node_loads"] = False
    if args.plain_first is not None:
        options["plain_first_polls"] = bool(args.plain_first)
    if args.look_ahead is not None:
        options["look_ahead"] = args.look_ahead == "1"
    if args.no_publish:
        options["publish_values"] = False
    if args.no_pipeline:
        options["pipeline_fetch"] = False
    if args.slots:
        options["gather_messages"] = False
        options["tile_rows"] = None
        options.setdefault("resident_waves_per_cu", options.get("task_lanes"))
    if work.kind == "sptrsv_csc":
        return sptrsv.compile_sptrsv_csc(**options)
    if work.kind == "sptrsv_csr":
        return sptrsv.compile_sptrsv_csr(**options)
    if args.auto:
        # the reference's demo fixes level launches with 128 threads; here the
        # scheduler decides
        options.setdefault("execution_mode", None)
        options.setdefault("threads_per_block", None)
    return spilu0.compile_ilu0_csr(**options)


def cpu_baseline(work, seconds):
    """The C restatement of the reference loop (oracle) on one host core."""
    from oracle import lcd_oracle
    lcd_oracle.lib()
    runs, elapsed = 0, 0.0
    start = time.perf_counter()
    while True:
        if work.kind == "sptrsv_csc":
            lcd_oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                  work.rhs, work.n)
        elif work.kind == "sptrsv_csr":
            lcd_oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                  work.rhs, work.n)
        else:
            lcd_oracle.ilu0_csr(work.data, work.indices, work.indptr)
        runs += 1
        elapsed = time.perf_counter() - start
        if elapsed >= seconds or runs >= 1000:
            break
    per_solve = elapsed / runs
    return {
        "value": round(work.algorithmic_bytes / per_solve / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "solve_ms": round(per_solve * 1e3, 3),
        "sample": f"{runs} full solves of {work.name} by the single-threaded "
                  "C restatement (gcc -O2, no FMA) of the reference loop",
        "host_cores_available": os.cpu_count(),
    }


PYTHON_LOOP_SECONDS = 1.5


def python_loop_baseline(work, seconds=PYTHON_LOOP_SECONDS):
    """The undecorated Python loop of the configuration (README.md:85-92,
    compiler/demo/sptrsv.py:26-43, compiler/demo/spilu0.py:21-47, the loops
    the reference's own end-to-end tests run on the host,
    compiler/e2e_tests/test_spilu0_e2e.py:19-70) on the leading tasks, for
    about ``seconds`` on one core, projected to the whole problem by the
    entries visited (the cost per entry does not change along these
    structures).  Lists instead of arrays: the loop a user would write over
    NumPy arrays is several times slower still."""
    n = work.n
    ptr, idx = work.indptr.tolist(), work.indices.tolist()
    val = work.data.tolist()
    deadline = time.perf_counter() + seconds
    start = time.perf_counter()
    rows = 0
    if work.kind == "sptrsv_csc":
        rhs = work.rhs.tolist()
        x = [0.0] * n
        for i in range(n):
            x[i] = (rhs[i] - x[i]) / val[ptr[i]]
            for j in range(ptr[i] + 1, ptr[i + 1]):
                x[idx[j]] += val[j] * x[i]
            rows = i + 1
            if (i & 1023) == 0 and time.perf_counter() > deadline:
                break
    elif work.kind == "sptrsv_csr":
        rhs = work.rhs.tolist()
        x = [0.0] * n
        for i in range(n):
            x[i] = rhs[i]
            for j in range(ptr[i], ptr[i + 1] - 1):
                x[i] -= val[j] * x[idx[j]]
            x[i] /= val[ptr[i + 1] - 1]
            rows = i + 1
            if (i & 1023) == 0 and time.perf_counter() > deadline:
                break
    else:
        for i in range(n):
            row_start, row_end = ptr[i], ptr[i + 1]
            for k_ptr in range(row_start, row_end):
                k = idx[k_ptr]
                if k >= i:
                    break
                diag_val = 0.0
                for diag_ptr in range(ptr[k], ptr[k + 1]):
                    if idx[diag_ptr] == k:
                        diag_val = val[diag_ptr]
                        break
                if diag_val != 0.0:
                    val[k_ptr] = val[k_ptr] / diag_val
                    l_ik = val[k_ptr]
                    for j_ptr in range(k_ptr + 1, row_end):
                        j = idx[j_ptr]
                        for kj_ptr in range(ptr[k], ptr[k + 1]):
                            if idx[kj_ptr] == j:
                                val[j_ptr] = val[j_ptr] - l_ik * val[kj_ptr]
                                break
            rows = i + 1
            if (i & 255) == 0 and time.perf_counter() > deadline:
                break
    elapsed = time.perf_counter() - start
    entries = max(ptr[rows], 1)
    return {"rows": rows, "entries": entries, "seconds": round(elapsed, 4),
            "cores": 1,
            "projected_full_ms": round(elapsed / entries * ptr[n] * 1e3, 1),
            "note": "the undecorated loop in CPython over lists, one core, "
                    f"leading {rows} of {n} iterations, projected by entries; "
                    "numba is not installed on this image"}


def latency_bounds(levels, arch):
    """What the dependences alone cost, in ms: ``levels`` dependent tasks one
    after the other with the hand-off free (``registers``: the chain of
    fp64 steps measured in one lane -- a bound under every executor, the
    walkers and the grid sweep included), with the hop between wavefronts of
    one workgroup through LDS (``lds``: tiles), and with the hop between
    workgroups through memory (``memory``: the flat queue, level launches).
    ``bound`` is the smallest."""
    chain = float(arch.get("chain_step_s", 0.0) or 0.0)
    lds = float(arch.get("lds_handoff_s", 0.0) or 0.0)
    memory = float(arch.get("handoff_s", 0.0) or 0.0)
    bounds = {"registers": levels * chain * 1e3,
              "lds": levels * (chain + lds) * 1e3,
              "memory": levels * (chain + memory) * 1e3}
    bounds["bound"] = min(bounds.values())
    return {key: round(value, 5) for key, value in bounds.items()}


def oracle_result(work):
    from oracle import lcd_oracle
    if work.kind == "sptrsv_csc":
        return lcd_oracle.sptrsv_csc(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
    if work.kind == "sptrsv_csr":
        return lcd_oracle.sptrsv_csr(work.indptr, work.indices, work.data,
                                     work.rhs, work.n)
    return lcd_oracle.ilu0_csr(work.data, work.indices, work.indptr)


def run_configuration(config, args, device, steps, warmup, arch,
                      cpu_seconds, python_loop=True):
    """Time one configuration; returns its record (see the module text)."""
    from lcd_amd import workloads
    from lcd_amd.dag_codegen import build_device_dag
    t0 = time.perf_counter()
    work = workloads.configuration(config)
    generate_s = time.perf_counter() - t0

    solver = build_solver(work, args, config)
    t0 = time.perf_counter()
    if work.kind == "ilu0_csr":
        pristine = device.to_device(work.data)
        operands = [device.to_device(work.data),
                    device.to_device(work.indices),
                    device.to_device(work.indptr)]
        scalars = []
    else:
        pristine = None
        operands = [device.to_device(a) for a in
                    (work.indptr, work.indices, work.data, work.rhs)]
        scalars = [work.n]
    upload_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    call = solver.bind(*operands, *scalars)
    device.synchronize()
    inspect_s = time.perf_counter() - t0
    schedule = solver.current_schedule
    plan = solver.schedule_plan(*operands, *scalars)
    lowering = solver.hip_lowering

    def step():
        if work.kind == "ilu0_csr":
            device.copy(operands[0], pristine)   # factorisation is in place
        call.launch(use_graph=not args.no_graph)

    t0 = time.perf_counter()
    step()
    call.synchronize()
    first_call_s = time.perf_counter() - t0
    # a long run (the chain of configuration 5 takes seconds per step) says
    # so once a minute on stderr; the timed region itself is not touched
    finished = threading.Event()

    def heartbeat():
        began = time.perf_counter()
        while not finished.wait(60.0):
            print(f"bench: {config} still running after "
                  f"{time.perf_counter() - began:.0f} s "
                  f"(first step took {first_call_s:.2f} s)",
                  file=sys.stderr, flush=True)

    threading.Thread(target=heartbeat, daemon=True).start()
    for _ in range(warmup):
        step()
    call.synchronize()
    start, stop = device.event(), device.event()
    device.record(start)
    for _ in range(steps):
        step()
    device.record(stop)
    elapsed_ms = device.elapsed_ms(start, stop)
    call.synchronize()
    finished.set()
    ms_per_step = elapsed_ms / steps

    launches_per_step = (plan.dag.levels
                         if schedule.execution_mode == "wavefront" else 1)
    gbps = work.algorithmic_bytes / (ms_per_step * 1e-3) / 1e9
    tile_rows = getattr(lowering, "tile_rows", None)
    record = {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "config": {
            "workload": work.name, "kind": work.kind, "n": work.n,
            "nnz": work.nnz, "levels": plan.dag.levels,
            "dag_edges": plan.dag.edges, "seed": work.seed,
            "execution_mode": schedule.execution_mode,
            "threads_per_block": schedule.threads_per_block,
            "task_lanes": lowering.task_lanes,
            "thread_unroll": schedule.thread_unroll,
            "dependence_protocol": lowering.dependence_protocol,
            "tile_rows": tile_rows,
            "tile_box": (list(plan.tile_boxes[1])
                         if getattr(plan, "tile_boxes", None) else None),
            "band_walker": bool(getattr(plan, "band_walker", False)),
            "level_walker": bool(getattr(plan, "level_walker", 0)),
            "grid_sweep": (list(plan.grid_sweep)
                           if getattr(plan, "grid_sweep", None) else None),
            "replayed_from_graph": not args.no_graph,
        },
        "roofline_pct": round(100.0 * gbps / HBM_PEAK_GBPS, 3),
        "algorithmic_bytes": work.algorithmic_bytes,
        "setup": {
            "generate_s": round(generate_s, 3), "upload_s": round(upload_s, 3),
            "inspect_compile_bind_s": round(inspect_s, 3),
            "first_call_s": round(first_call_s, 4),
            # code objects found on disk / compiled by hiprtc so far in this
            # process (a second process finds them all)
            "code_cache": dict(hip_runtime_module().code_cache_statistics),
        },
    }
    # the on-device inspector alone (edges, counts, level sets and, for the
    # mailbox protocol, the incoming listing), operands resident
    names = solver.dag_plan.arguments
    values = dict(zip(names, list(operands) + scalars))
    if work.kind == "ilu0_csr":
        values["n"] = work.n
    mailbox = lowering.dependence_protocol == "mailbox"
    inspector = []
    for _ in range(1 if config == "c5" else 3):
        device.synchronize()
        t0 = time.perf_counter()
        dag = build_device_dag(solver.dag_plan, values, device, levels=True,
                               incoming=mailbox)
        device.synchronize()
        inspector.append(time.perf_counter() - t0)
        dag.destroy()
    record["setup"]["inspector_ms"] = round(min(inspector) * 1e3, 3)
    record["gflops"] = round(
        work.true_flops / (ms_per_step * 1e-3) / 1e9, 3)
    record["true_flops"] = int(work.true_flops)
    record["gflops_reference_formula"] = round(
        work.reference_style_flops / (ms_per_step * 1e-3) / 1e9, 3)

    kernel_ms = ms_per_step / launches_per_step
    if schedule.execution_mode == "sync_free":
        # the persistent executor is one launch per step: time that launch
        # alone with HIP events on the library stream (eager launches, so the
        # events sit directly around the kernel; the step above also holds
        # the reset and operand-staging kernels)
        device.kernel_timing = {"name": lowering.kernel_name}
        try:
            for _ in range(min(steps, 20)):
                if work.kind == "ilu0_csr":
                    device.copy(operands[0], pristine)
                call.launch(use_graph=False)
            call.synchronize()
            pairs = device.kernel_timing.get("events", [])
            if pairs:
                # (around a kernel of a few tens of microseconds the events of
                # an eager launch also see the launch itself: the kernel takes
                # no longer than the replayed step that contains it)
                kernel_ms = min(kernel_ms, sum(
                    device.elapsed_ms(a, b) for a, b in pairs) / len(pairs))
        finally:
            device.kernel_timing = None
    bytes_per_launch = work.algorithmic_bytes / launches_per_step
    achieved = bytes_per_launch / (kernel_ms * 1e-3) / 1e9
    key = traffic_key(config, schedule.execution_mode,
                      lowering.dependence_protocol, lowering.task_lanes,
                      tile_rows,
                      plan.tile_boxes[1] if getattr(plan, "tile_boxes", None)
                      else None,
                      "band_walker" if getattr(plan, "band_walker", False)
                      else "level_walker" if getattr(plan, "level_walker", 0)
                      else "grid_sweep" if getattr(plan, "grid_sweep", None)
                      else False)
    record["roofline"] = {
        "bound": "hbm", "achieved": round(achieved, 3), "peak": HBM_PEAK_GBPS,
        "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 6),
        "traffic": measured_traffic(key),
        "traffic_key": key,
        "kernel": lowering.kernel_name,
        "launches_per_step": launches_per_step,
        "avg_launch_ms": round(kernel_ms, 6),
        "dependency_levels": plan.dag.levels,
        # what the dependences alone cost (see latency_bounds): the floor is
        # the chain of dependent fp64 tasks with every hand-off free; the
        # figures with a hop per level say what each kind of executor pays
        "handoff_us": {"memory": round(arch["handoff_s"] * 1e6, 4),
                       "lds": round(arch["lds_handoff_s"] * 1e6, 4),
                       "registers": round(arch["chain_step_s"] * 1e6, 4)},
    }
    bounds = latency_bounds(plan.dag.levels, arch)
    record["roofline"]["latency_bound_ms"] = bounds.pop("bound")
    record["roofline"]["latency_by_handoff_ms"] = bounds
    record["roofline"]["latency_bound_holds"] = bool(
        record["roofline"]["latency_bound_ms"] <= ms_per_step)

    if not args.no_check:
        expected = oracle_result(work)
        if work.kind == "ilu0_csr":
            call.synchronize()
            got = operands[0].copy_to_host()
        else:
            got = call.result()
        error = elementwise_error(got, expected)
        record["max_rel_error_vs_oracle"] = error
        record["bit_identical_to_sequential_loop"] = bool(
            np.array_equal(got, expected))
        record["parity_ok"] = bool(error <= RTOL)
        del got, expected
    if not args.no_cpu:
        if cpu_seconds > 0:
            record["cpu_baseline"] = cpu_baseline(work, cpu_seconds)
        if python_loop:
            record["cpu_python_loop"] = python_loop_baseline(work)
    # release the device memory of this configuration before the next one
    del call, plan, solver, operands, pristine, values, work
    gc.collect()
    device.synchronize()
    return record


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--config", default=None,
                        choices=["c1", "c2", "c3", "c4", "c5"],
                        help="time this configuration only (default: "
                             "configuration 2 as the headline plus a record "
                             "for every configuration)")
    parser.add_argument("--mode", default=None)
    parser.add_argument("--tpb", type=int, default=None)
    parser.add_argument("--lanes", type=int, default=None)
    parser.add_argument("--unroll", type=int, default=None)
    parser.add_argument("--protocol", default=None)
    parser.add_argument("--waves-per-cu", dest="waves_per_cu", type=float,
                        default=None)
    parser.add_argument("--spin-sleep", dest="spin_sleep", type=int,
                        default=None)
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--tile-rows", dest="tile_rows", type=int, default=None,
                        help="tiled persistent executor: rows per tile")
    parser.add_argument("--tile-positions", dest="tile_positions", type=int,
                        default=None,
                        help="tiled published pull (ILU0): entries of the "
                             "publication buffer a tile mirrors in LDS")
    parser.add_argument("--band-walker", dest="band_walker", type=int,
                        default=None, choices=(0, 1),
                        help="1: run chain-like DAGs on one wavefront in "
                             "program order; 0: never (default: per plan)")
    parser.add_argument("--level-walker", dest="level_walker", type=int,
                        default=None, choices=(0, 1),
                        help="1: run small DAGs with narrow levels on one "
                             "wavefront, a level per step; 0: never (default: "
                             "per plan)")
    parser.add_argument("--grid-sweep", dest="grid_sweep", type=int,
                        default=None, choices=(0, 1),
                        help="1: run axis stencils on a 3-D grid on the grid "
                             "sweep (a lane per grid line); 0: never "
                             "(default: per plan)")
    parser.add_argument("--sweep-shape", dest="sweep_shape", default=None,
                        help="grid sweep: WY,GY,GZ,SKZ (lines of a bundle "
                             "along y, bundles of a workgroup along y and z, "
                             "steps between the z rows of a bundle)")
    parser.add_argument("--tile-box", dest="tile_box", default=None,
                        help="tiles over boxes of a structured grid: "
                             "'auto', 'none' or extents as 32x8x16")
    parser.add_argument("--segment-capacity", dest="segment_capacity",
                        type=int, default=None,
                        help="entries of a task's own segment staged in LDS")
    parser.add_argument("--level-gather", dest="level_gather",
                        action="store_true",
                        help="level launches gather incoming products "
                             "instead of pushing them with atomics")
    parser.add_argument("--slots", action="store_true",
                        help="message slots instead of the gathered form of "
                             "the mailbox protocol (implies no tiles)")
    parser.add_argument("--auto", action="store_true",
                        help="let the analytic scheduler choose the schedule "
                             "instead of the tuned defaults")
    parser.add_argument("--no-queue-loads", action="store_true",
                        help="read structure arrays through the task id "
                             "instead of copies in task order")
    parser.add_argument("--plain-first", type=int, default=None,
                        help="1: poll a producer's value with a plain load "
                             "and confirm only the empty marker coherently")
    parser.add_argument("--look-ahead", default=None,
                        choices=("0", "1"),
                        help="published pull: locate the next producer's "
                             "values while waiting for this one's (default 1)")
    parser.add_argument("--no-publish", action="store_true",
                        help="pull on a sequential loop through done flags")
    parser.add_argument("--no-pipeline", action="store_true",
                        help="tiled mailbox: load a round's records and "
                             "operands when the round starts")
    parser.add_argument("--no-graph", action="store_true",
                        help="issue every launch of a step eagerly instead "
                             "of replaying the captured graph")
    parser.add_argument("--no-cpu", action="store_true")
    parser.add_argument("--no-check", action="store_true")
    parser.add_argument("--arch", action="store_true",
                        help="also report every measured machine constant")
    args = parser.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this path (one sparse triangular "
              "DAG) runs on a single MI355X; --gpus must be 1.",
              file=sys.stderr)
        return 2
    overrides = {name: os.environ[name] for name in OVERRIDE_VARIABLES
                 if os.environ.get(name)}
    if overrides:
        print(f"bench: generated kernels are modified by {overrides}; the "
              "record says so", file=sys.stderr)

    from lcd_amd import hip_runtime
    device = hip_runtime.default_device()
    arch = device.measure_arch()

    headline = args.config or "c2"
    everything = args.config is None
    head = run_configuration(headline, args, device, args.steps, args.warmup,
                             arch, args.cpu_seconds)
    result = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f64",
        "data": "synthetic",
        "config": head["config"],
        "solve_ms": head["ms_per_step"],
    }
    for key, value in head.items():
        result.setdefault(key, value)
    result["kernel_overrides"] = overrides or None
    result["error_measure"] = (
        "max_i |x_i - ref_i| / (|ref_i| + 1e-3 max|ref|) against the "
        "sequential loop; passes at <= 1e-12")
    failed = [] if head.get("parity_ok", True) else [headline]
    if everything:
        sub_args = argparse.Namespace(**vars(args))
        for name in ("mode", "tpb", "lanes", "unroll", "protocol",
                     "waves_per_cu", "spin_sleep", "tile_rows",
                     "plain_first", "look_ahead", "tile_positions",
                     "segment_capacity", "tile_box", "band_walker",
                     "level_walker", "grid_sweep", "sweep_shape"):
            setattr(sub_args, name, None)
        for name in ("slots", "no_queue_loads", "no_publish", "no_pipeline",
                     "no_graph", "level_gather"):
            setattr(sub_args, name, False)
        records = {}
        for config in ("c1", "c2", "c3", "c4", "c5"):
            if config == headline and vars(sub_args) == vars(args):
                records[config] = dict(head)
                continue
            print(f"bench: {config}", file=sys.stderr, flush=True)
            steps, warmup = SUB_STEPS[config]
            records[config] = run_configuration(
                config, sub_args, device, steps, warmup, arch,
                CPU_SECONDS_SUB)
        # configuration 2 under the level-launched executor, the mode
        # BASELINE.json names for it (one captured graph of `levels` launches)
        print("bench: c2 wavefront", file=sys.stderr, flush=True)
        sub_args.mode = "wavefront"
        records["c2_wavefront"] = run_configuration(
            "c2", sub_args, device, 20, 3, arch, 0.0, python_loop=False)
        # ILU0 under level launches with 128 threads per block, the mode and
        # block size the reference's demo fixes
        # (compiler/demo/spilu0.py:85-98)
        print("bench: c4 wavefront", file=sys.stderr, flush=True)
        records["c4_wavefront"] = run_configuration(
            "c4", sub_args, device, 5, 1, arch, 0.0, python_loop=False)
        result["configs"] = records
        failed += [name for name, record in records.items()
                   if not record.get("parity_ok", True)]
    if args.arch or everything:
        result["arch_constants"] = arch
    print(json.dumps(result))
    if failed:
        print(f"parity check failed for {failed}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""The ``parallel`` decorator: LCD's `@parallel` on an MI355X backend.

Same contract as compiler/decorator.py:138-528 of the reference: identical
keyword arguments (``loop``/``block_map``/``block_loop``, ``function_props``,
``execution_mode``, ``threads_per_block``, ``thread_loop``/``thread_map``,
``thread_unroll``/``thread_unroll_factor``, ``n_warp``,
``dependence_protocol``, ``scheduler``, ``arch_constants``,
``sync_free_ready_count``, ``validate_dag_endpoints``, ``band_width``), the
wrapper is called with ordinary host values and returns what the original
``return`` returns, and the same introspection attributes are published
(``cuda_*`` names are kept as aliases of the ``hip_*`` ones).

What happens underneath is different: dependences come from
``lcd_amd.dependence`` (or explicit ``edge_rules=``), the inspector runs on
the GPU, plans keep the structure arrays and the DAG resident in HBM, kernels
are HIP C++ compiled with hiprtc, and repeated calls replay a hipGraph.
Extra keyword arguments: ``task_lanes`` (lanes per task, power of two <= 64),
``edge_rules`` (explicit :class:`SegmentRule` list), ``device`` (device
layer), ``verbose`` (print generated sources like the reference does).
"""

import ast
import functools
from dataclasses import replace
import inspect
import textwrap

import numpy as np

from lcd_amd import hip_runtime
from lcd_amd.dag_codegen import (
    COUNTER_DEPENDENCE,
    MAILBOX_DEPENDENCE,
    PULL_DEPENDENCE,
    PUSH_DEPENDENCE,
    build_device_dag,
    compile_dag_builder,
    create_dag_plan,
    direct_dependence,
    generate_dag_source,
)
from lcd_amd.dag_preprocessing import (
    attach_auxiliary_values,
    execution_data_from_device_dag,
)
from lcd_amd.dependence import DependenceAnalysis, analyze_dependences
from lcd_amd.hip_emitter import (
    HIPLoweringError,
    LEVEL_WALKER_ARGUMENTS,
    LEVEL_WALKER_ENTRIES,
    LEVEL_WALKER_TASKS,
)
from lcd_amd.hip_lowering import lower_to_hip
from lcd_amd.hip_runtime import (
    compile_hip_module,
    evaluate_host_prelude,
    execute_hip_call,
    launch_hip_call,
    prepare_hip_arguments,
)
from lcd_amd.scheduler import (
    AUTO,
    SYNC_FREE,
    WAVEFRONT,
    AnalyticScheduler,
    CalibratedScheduler,
    SchedulePlan,
    BAND_WALKER_THREADS_PER_BLOCK,
    GRID_SWEEP_SHAPE,
    PAIR_TABLE_ENTRIES_PER_POSITION,
    PUBLISHED_TILE_MIN_LOCALITY,
    PUBLISHED_TILE_POSITIONS,
    PUBLISHED_TILE_THREADS_PER_BLOCK,
    TILE_BOX_THREADS_PER_BLOCK,
    TILE_THREADS_PER_BLOCK,
    automatic_tile_box,
    band_walker_applies,
    level_walker_records,
    sequential_advice,
    SchedulerAdvice,
    automatic_tile_rows,
    structured_grid,
    automatic_tile_threads,
    ScheduleSpace,
    count_inner_loop_flops,
    extract_workload_features,
    inspection_fingerprint,
    pointer_array_names,
    segment_trip_counts,
    compile_thread_trip_counter,
    TRIP_PROBE_SAMPLE,
    measure_thread_trip_counts,
)
from lcd_amd.hip_grid_sweep import (
    SWEEP_MAX_LINE,
    sweep_applies,
    sweep_geometry,
)
from lcd_amd.structural_lookups import (
    create_structural_lookup_plan,
    materialize_structural_lookups,
    structural_argument_names,
)

SCHEDULE_CACHE_SIZE = 8
VARIANT_ATTRIBUTES = (
    "hip_lowering", "compiled_hip_module", "hip_kernel", "hip_launcher",
    "hip_source", "hip_kernel_source", "hip_launcher_ast",
    "hip_launcher_source",
    # names the reference publishes
    "cuda_lowering", "compiled_cuda_module", "cuda_kernel", "cuda_launcher",
    "cuda_module_ast", "cuda_kernel_ast", "cuda_source", "cuda_kernel_source",
    "cuda_launcher_ast", "cuda_launcher_source",
)


def _variant_attributes(lowering, compiled):
    return {
        "hip_lowering": lowering,
        "compiled_hip_module": compiled,
        "hip_kernel": lowering.kernel_name,
        "hip_launcher": compiled.launcher,
        "hip_source": lowering.source,
        "hip_kernel_source": lowering.kernel_source,
        "hip_launcher_ast": lowering.launcher_ast,
        "hip_launcher_source": lowering.launcher_source,
        "cuda_lowering": lowering,
        "compiled_cuda_module": compiled,
        "cuda_kernel": lowering.kernel_name,
        "cuda_launcher": compiled.launcher,
        "cuda_module_ast": None,
        "cuda_kernel_ast": None,
        "cuda_source": lowering.source,
        "cuda_kernel_source": lowering.kernel_source,
        "cuda_launcher_ast": lowering.launcher_ast,
        "cuda_launcher_source": lowering.launcher_source,
    }


def _function_source(function):
    source = textwrap.dedent(inspect.getsource(function))
    return "\n".join(line for line in source.splitlines()
                     if not line.startswith("@"))


def parallel(**kwargs):
    def decorator(function):
        loop = kwargs.get("loop", kwargs.get("block_map",
                                             kwargs.get("block_loop")))
        if loop is None:
            raise ValueError(
                "parallel requires a block-mapped iterator via `loop`, "
                "`block_map`, or `block_loop`.")
        function_props = kwargs.get("function_props", {})
        verbose = kwargs.get("verbose", False)
        source = _function_source(function)
        if verbose:
            print(source)
        function_ast = ast.parse(source)
        structural_lookups = create_structural_lookup_plan(
            function_ast, function_props)
        if kwargs.get("edge_rules") is not None:
            dependence_analysis = DependenceAnalysis(
                ordering_dependences=list(kwargs["edge_rules"]))
        else:
            dependence_analysis = analyze_dependences(
                function_ast, loop, function_props,
                strict=kwargs.get("strict_dependences", False))
            if dependence_analysis.conservative:
                import warnings
                kept = [str(d) for d in dependence_analysis.kept_dependences
                        if getattr(d.rule, "relation", 0) == 2]
                warnings.warn(
                    f"@parallel({function.__name__}): a dependence could be "
                    "neither refuted nor enumerated and is kept as the "
                    "complete order (the iterations run one after the "
                    "other): " + "; ".join(kept) + ".  Pass edge_rules= to "
                    "state the dependences, or strict_dependences=True to "
                    "get an error instead.", stacklevel=2)
        if verbose:
            for dependence in dependence_analysis.raw_dependences:
                print(dependence)
            for rule in dependence_analysis.ordering_dependences:
                print(rule.describe())
            print("Reduction dependences:")
            for text in dependence_analysis.reduction_dependences:
                print(text)

        signature = inspect.signature(function)
        argument_names = list(signature.parameters)
        execution_mode = kwargs.get("execution_mode", AUTO)
        thread_loop = kwargs.get("thread_loop", kwargs.get("thread_map"))
        thread_unroll = kwargs.get("thread_unroll",
                                   kwargs.get("thread_unroll_factor"))
        space_options = dict(
            execution_mode=execution_mode,
            threads_per_block=kwargs.get("threads_per_block"),
            thread_unroll=thread_unroll,
            thread_mapped=thread_loop is not None,
            n_warp=kwargs.get("n_warp"),
            task_lanes=kwargs.get("task_lanes"),
        )
        band_width = kwargs.get("band_width", 1)
        if band_width == 1:
            space_options["level_gather"] = kwargs.get("level_gather", True)
        scheduler = kwargs.get("scheduler") or CalibratedScheduler(
            kwargs.get("arch_constants"))
        device_layer = kwargs.get("device")
        lowered_variants = {}
        compiled_variants = {}
        dependence = None

        def get_device():
            return device_layer or hip_runtime.default_device()

        tile_option = kwargs.get("tile_rows", "auto")
        if not (tile_option in (None, "auto") or (
                isinstance(tile_option, int) and tile_option >= 0)):
            raise ValueError(
                "tile_rows must be None, 'auto' or a positive integer.")

        tile_box_option = kwargs.get("tile_box", "auto")
        if not (tile_box_option in (None, "auto") or (
                isinstance(tile_box_option, (tuple, list))
                and len(tile_box_option) == 3
                and all(isinstance(extent, int) and extent > 0
                        for extent in tile_box_option))):
            raise ValueError(
                "tile_box must be None, 'auto' or three positive integers.")

        walker_option = kwargs.get("band_walker", "auto")
        if walker_option not in ("auto", True, False):
            raise ValueError("band_walker must be 'auto', True or False.")
        level_option = kwargs.get("level_walker", "auto")
        if level_option not in ("auto", True, False):
            raise ValueError("level_walker must be 'auto', True or False.")

        sweep_option = kwargs.get("grid_sweep", "auto")
        if sweep_option not in ("auto", True, False):
            raise ValueError("grid_sweep must be 'auto', True or False.")
        sweep_shape = tuple(kwargs.get("sweep_shape", GRID_SWEEP_SHAPE))
        if len(sweep_shape) != 4:
            raise ValueError(
                "sweep_shape must be (WY, GY, GZ, SKZ): lines of a bundle "
                "along y, bundles of a workgroup along y and z, steps "
                "between the z rows of a bundle.")

        registers_option = kwargs.get("segment_registers", "auto")
        if registers_option not in ("auto", True, False):
            raise ValueError("segment_registers must be 'auto', True or False.")

        def lower_variant(lowering_key, tile_rows=None, single_chunk=False,
                          task_records=True, by_position=False,
                          registers=False, walker=False, level=0, sweep=None):
            variant_key = (lowering_key, tile_rows, single_chunk, task_records,
                           by_position, registers, walker, level, sweep)
            if variant_key not in lowered_variants:
                (mode, threads_per_block, unroll, n_warp, protocol,
                 task_lanes) = lowering_key
                lowered_variants[variant_key] = lower_to_hip(
                    function_ast,
                    loop_iterator=loop,
                    reductions=dependence_analysis,
                    execution_mode=mode,
                    sync_free_ready_count=kwargs.get(
                        "sync_free_ready_count", 0),
                    wavefront_threads_per_block=threads_per_block,
                    thread_loop_iterator=thread_loop,
                    thread_unroll_factor=unroll,
                    n_warp=n_warp if thread_loop is not None else None,
                    dependence_protocol=protocol,
                    direct_dependence=(
                        None if protocol == COUNTER_DEPENDENCE else dependence),
                    function_props=function_props,
                    structural_lookups=structural_lookups,
                    task_lanes=task_lanes or None,
                    chain_tasks=band_width != 1,
                    resident_waves_per_cu=kwargs.get("resident_waves_per_cu"),
                    # a nap between polls spares the memory pipeline where
                    # polls go to memory; in tiles they go to LDS and the nap
                    # is only delay (128^3 grid 0.250 -> 0.237 ms, the 4 M-row
                    # chain 1.86 -> 1.79 s without it)
                    spin_sleep=kwargs.get("spin_sleep", 0 if tile_rows else 1),
                    **({"spin_limit": kwargs["spin_limit"]}
                       if "spin_limit" in kwargs else {}),
                    value_flags=kwargs.get("value_flags", True),
                    gather_messages=kwargs.get("gather_messages", True),
                    segment_cache=kwargs.get("segment_cache", True),
                    tile_rows=tile_rows if mode == SYNC_FREE else None,
                    task_records=(task_records
                                  and kwargs.get("task_records", True)),
                    single_chunk=single_chunk,
                    queue_node_loads=kwargs.get("queue_node_loads", True),
                    plain_first_polls=kwargs.get("plain_first_polls"),
                    publish_values=kwargs.get("publish_values", True),
                    look_ahead=kwargs.get("look_ahead", True),
                    segment_capacity=kwargs.get("segment_capacity"),
                    pipeline_fetch=kwargs.get("pipeline_fetch", True),
                    tile_positions=kwargs.get("tile_positions"),
                    tile_by_position=by_position,
                    segment_registers=bool(registers),
                    pair_tables=registers == 2,
                    band_walker=walker,
                    level_walker=level,
                    grid_sweep=sweep,
                    prepared_division=kwargs.get("prepared_division", True),
                    watchdog_seconds=kwargs.get("watchdog_seconds"),
                    level_records=kwargs.get("level_records", True),
                    full_fences=kwargs.get("full_fences", False),
                    dynamic_fetch=kwargs.get("dynamic_fetch", False),
                )
            return lowered_variants[variant_key]

        def compile_variant(lowering_key, tile_rows=None, single_chunk=False,
                            task_records=True, by_position=False,
                            registers=False, walker=False, level=0,
                            sweep=None):
            lowering = lower_variant(lowering_key, tile_rows, single_chunk,
                                     task_records, by_position, registers,
                                     walker, level, sweep)
            variant_key = (lowering_key, tile_rows, single_chunk, task_records,
                           by_position, registers, walker, level, sweep)
            if variant_key not in compiled_variants:
                compiled_variants[variant_key] = compile_hip_module(
                    lowering, function_globals=function.__globals__)
            return lowering, compiled_variants[variant_key]

        def segment_lengths(pointer_name, values):
            """(longest, mean) segment length of a pointer array of this
            structure, or None when the array is not among the values."""
            pointers = values.get(pointer_name)
            if pointers is None:
                return None
            if hip_runtime.is_device_array(pointers):
                pointers = pointers.copy_to_host()
            lengths = np.diff(np.asarray(pointers))
            if len(lengths) == 0:
                return 0, 0.0
            return int(lengths.max()), float(lengths.mean())

        def tiles_for(dag, schedule, values):
            """(schedule, tile_rows): the tiled persistent executor when it
            is asked for, or pays for this DAG, and the loop allows it."""
            if (schedule.execution_mode != SYNC_FREE or band_width != 1
                    or not tile_option):
                return schedule, None
            rows = (tile_option if isinstance(tile_option, int)
                    else automatic_tile_rows(dag))
            if not rows:
                return schedule, None
            tiled = schedule
            tile_threads = automatic_tile_threads(dag)
            if (tile_option == "auto" and thread_loop is not None
                    and kwargs.get("threads_per_block") is None
                    and not tile_threads % max(schedule.task_lanes, 1)):
                tiled = replace(schedule, threads_per_block=tile_threads)
            variant = lower_variant(tiled.lowering_key, rows)
            if variant.tile_rows is None:
                return schedule, None        # tiles do not apply to this loop
            if tile_option == "auto" and variant.published_array is not None:
                # published pull (ILU0): tiles pay with many wavefronts per
                # tile, rows short enough to live in registers, a tile whose
                # slice of the publication buffer fits the LDS copy, and a
                # structure in which consecutive rows depend on each other
                # (9-point 1024^2 grid: 4.1 against 5.4 ms; 38 ms at the
                # sizes chosen for SpTRSV)
                if registers_option is False:
                    return schedule, None
                stats = segment_lengths(variant.segment_pointer, values)
                if stats is None or stats[0] > 64 or stats[1] <= 0:
                    return schedule, None
                rows = int(0.9 * PUBLISHED_TILE_POSITIONS / stats[1])
                rows = max(64, min(rows, 2048))
                if (dag.n < 4 * rows
                        or dag.tile_locality(rows) < PUBLISHED_TILE_MIN_LOCALITY):
                    return schedule, None
                tiled = schedule
                if (kwargs.get("threads_per_block") is None
                        and not PUBLISHED_TILE_THREADS_PER_BLOCK
                        % max(schedule.task_lanes, 1)):
                    tiled = replace(schedule, threads_per_block=(
                        PUBLISHED_TILE_THREADS_PER_BLOCK))
                variant = lower_variant(tiled.lowering_key, rows)
                if variant.tile_rows is None:
                    return schedule, None
            return tiled, rows

        def registers_for(schedule, rows, values, lookups, dag_rows):
            """(level, tables) for this plan.  Level 1: the tasks' own
            segments (ILU0's rows) live in registers -- the loop allows it
            and no segment of this structure has more than 64 entries.  Level
            2: the structure searches of the producer loop are read from
            tables as well (``pair_tables``, built here, at most
            PAIR_TABLE_ENTRIES_PER_POSITION entries per stored position).
            Level 0: neither."""
            if registers_option is False:
                return 0, {}
            # (level launches take the registers with the tables or not at
            # all: their task reads other segments through the tables only)
            level_launches = schedule.execution_mode == WAVEFRONT
            try:
                variant = lower_variant(schedule.lowering_key, rows,
                                        registers=2 if level_launches else 1)
            except HIPLoweringError:
                return 0, {}
            if not variant.segment_registers:
                return 0, {}
            stats = segment_lengths(variant.segment_pointer, values)
            if stats is None:
                return 0, {}
            longest = stats[0]
            if longest > 64:
                if registers_option is True:
                    raise ValueError(
                        "segment_registers=True needs segments of at most 64 "
                        f"entries; the longest has {longest}.")
                return 0, {}
            if not kwargs.get("pair_tables", True):
                return 0 if level_launches else 1, {}
            variant = lower_variant(schedule.lowering_key, rows, registers=2)
            if not variant.structure_tables:
                return 0 if level_launches else 1, {}
            device = get_device()
            tables = {}
            try:
                for entry in variant.structure_tables:
                    if entry[0] == "at":
                        _, name, lookup, index_array = entry
                        tables[name] = device.gather_int32(
                            lookups[lookup], values[index_array])
                    elif entry[0] == "start":
                        _, name, pointer_array, index_array = entry
                        tables[name] = device.gather_int32(
                            values[pointer_array], values[index_array])
                    else:
                        _, name, pointer_array, index_array = entry
                        positions = max(int(round(stats[1] * dag_rows)), 1)
                        entries = device.pair_lookup_entries(
                            values[pointer_array], values[index_array])
                        if entries > PAIR_TABLE_ENTRIES_PER_POSITION * positions:
                            return 0 if level_launches else 1, {}
                        tables["_lcd_pair_base"], tables[name] = (
                            device.pair_lookup_build(values[pointer_array],
                                                     values[index_array],
                                                     offsets=True))
            except (hip_runtime.HIPRuntimeError, KeyError):
                return 0 if level_launches else 1, {}
            return 2, tables

        def walker_for(dag, schedule):
            """(schedule, lowering) when this plan runs on the band walker:
            asked for with ``band_walker=True``, or chosen for a DAG that is
            close to a chain (unless the call fixes a tile size)."""
            if walker_option is False:
                return None
            forced = walker_option is True
            usable = (schedule.execution_mode == SYNC_FREE and band_width == 1
                      and schedule.lowering_key[4] in (MAILBOX_DEPENDENCE,
                                                       PULL_DEPENDENCE)
                      and (forced or not isinstance(tile_option, int)))
            if usable and not band_walker_applies(dag, forced=forced):
                usable = False
            candidate = schedule
            lowering = None
            if usable:
                # (the distributed loop is gone from the walker's kernel:
                # nothing to unroll)
                candidate = replace(schedule, thread_unroll=1)
                if kwargs.get("threads_per_block") is None:
                    candidate = replace(
                        candidate,
                        threads_per_block=BAND_WALKER_THREADS_PER_BLOCK)
                try:
                    lowering = lower_variant(candidate.lowering_key, None,
                                             False, False, False, 0, True)
                except HIPLoweringError:
                    if forced:
                        raise
                    usable = False
            if not usable:
                if forced:
                    raise ValueError(
                        "band_walker=True needs the persistent executor with "
                        "the mailbox or pull protocol (execution_mode="
                        "'sync_free', band_width=1) and a DAG whose edges all "
                        "span fewer than 64 iterations.")
                return None
            return candidate, lowering

        def level_walker_for(dag, schedule, build_incoming):
            """(schedule, lowering, dag, tables) when this plan runs on the
            level walker: a small DAG with narrow levels and few incoming
            entries per task (``level_walker=True`` asks for it, the
            default takes it unless the call fixes a tile size)."""
            if level_option is False:
                return None
            forced = level_option is True
            usable = (schedule.execution_mode == SYNC_FREE and band_width == 1
                      and schedule.lowering_key[4] in (MAILBOX_DEPENDENCE,
                                                       PULL_DEPENDENCE)
                      and (forced or not isinstance(tile_option, int))
                      and 0 < dag.n <= LEVEL_WALKER_TASKS and dag.edges > 0)
            records = lowering = None
            candidate = schedule
            if usable:
                if not incoming_positions:
                    dag = build_incoming()
                records = level_walker_records(dag, LEVEL_WALKER_TASKS,
                                               LEVEL_WALKER_ENTRIES,
                                               forced=forced)
                usable = records is not None
            if usable:
                candidate = replace(schedule, thread_unroll=1)
                if kwargs.get("threads_per_block") is None:
                    candidate = replace(
                        candidate,
                        threads_per_block=BAND_WALKER_THREADS_PER_BLOCK)
                try:
                    lowering = lower_variant(candidate.lowering_key, None,
                                             False, False, False, 0, False,
                                             records[0])
                except HIPLoweringError:
                    if forced:
                        raise
                    usable = False
            if not usable:
                if forced:
                    raise ValueError(
                        "level_walker=True needs the persistent executor with "
                        "the mailbox or pull protocol and a DAG of at most "
                        f"{LEVEL_WALKER_TASKS} tasks with at most "
                        f"{LEVEL_WALKER_ENTRIES} incoming entries each.")
                return None
            device = get_device()
            tables = {name: device.to_device(values) for name, values in zip(
                LEVEL_WALKER_ARGUMENTS, records[1:])}
            return candidate, lowering, dag, tables, records[0]

        def sweep_for(dag, schedule, build_incoming):
            """(schedule, lowering, dag, shape) when this plan runs on the
            grid sweep: the DAG is an axis stencil on a three-dimensional
            grid in natural order whose lines the sweep's face arrays hold
            (``grid_sweep=True`` asks for it; the default takes it for any
            such DAG beyond the level walker's size unless the call fixes a
            tile size)."""
            if sweep_option is False:
                return None
            forced = sweep_option is True
            usable = (schedule.execution_mode == SYNC_FREE and band_width == 1
                      and schedule.lowering_key[4] in (MAILBOX_DEPENDENCE,
                                                       PULL_DEPENDENCE)
                      and (forced or (not isinstance(tile_option, int)
                                      and dag.n > LEVEL_WALKER_TASKS))
                      and dag.edges > 0)
            grid = (kwargs.get("tile_grid") or structured_grid(dag)
                    if usable else None)
            shape = None
            if grid is not None:
                grid = tuple(int(extent) for extent in grid)
                if len(grid) == 3 and sweep_applies(grid, *sweep_shape):
                    shape = grid + sweep_shape
            lowering, candidate = None, schedule
            if shape is not None:
                geometry = sweep_geometry(grid, *sweep_shape)
                candidate = replace(schedule, thread_unroll=1,
                                    threads_per_block=geometry["threads"])
                try:
                    lowering = lower_variant(candidate.lowering_key, None,
                                             False, False, False, 0, False, 0,
                                             shape)
                except HIPLoweringError:
                    if forced:
                        raise
                    lowering = None
            if lowering is None:
                if forced:
                    raise ValueError(
                        "grid_sweep=True needs the persistent executor with "
                        "the mailbox or pull protocol and a DAG that is an "
                        "axis stencil on a three-dimensional grid in natural "
                        f"order with lines of at most {SWEEP_MAX_LINE} points.")
                return None
            if not incoming_positions:
                dag = build_incoming()
            return candidate, lowering, dag, shape

        def boxes_for(dag, schedule, rows):
            """(grid, box) when the tiles of this plan are boxes of a
            structured grid: asked for with ``tile_box``, the grid given as
            ``tile_grid`` or recognised from the DAG's edge offsets."""
            if not rows or tile_box_option is None:
                return None
            grid = kwargs.get("tile_grid") or structured_grid(dag)
            if grid is None:
                return None
            grid = tuple(int(extent) for extent in grid)
            box = (automatic_tile_box(grid, rows) if tile_box_option == "auto"
                   else tuple(tile_box_option))
            if box is None:
                return None
            points = box[0] * box[1] * box[2]
            try:
                variant = lower_variant(schedule.lowering_key, points, True,
                                        True, True)
            except HIPLoweringError:
                return None
            if not variant.tile_by_position or (
                    dag.n * variant.task_record_lanes >= 2 ** 31):
                return None
            return grid, box

        host_lowering = lower_variant(
            ScheduleSpace.from_options(**space_options).configurations()[0])
        dag_argument_names = argument_names + [
            name for name in host_lowering.lifted_loop_parameters
            if name not in argument_names]
        block_loop = host_lowering  # (lowering already validated the loop)
        loop_node = next(
            node for node in ast.walk(function_ast)
            if isinstance(node, ast.For) and isinstance(node.target, ast.Name)
            and node.target.id == loop)
        range_arguments = loop_node.iter.args
        node_lower = (ast.unparse(range_arguments[0])
                      if len(range_arguments) > 1 else "0")
        node_count = ast.unparse(
            range_arguments[1] if len(range_arguments) > 1
            else range_arguments[0])
        dag_plan = create_dag_plan(
            dependence_analysis.ordering_dependences, None,
            parallel_iterator=loop, arguments=dag_argument_names,
            function_props=function_props, node_count=node_count,
            node_lower=node_lower)
        validate_endpoints = kwargs.get("validate_dag_endpoints", False)
        dependence = direct_dependence(dag_plan, thread_loop,
                                       validate_endpoints=validate_endpoints)
        schedule_space = ScheduleSpace.from_options(
            **space_options,
            direct_protocol=None if dependence is None else dependence.kind,
            dependence_protocol=kwargs.get("dependence_protocol"),
            sequential_pull=bool(dependence is not None
                                 and dependence.sequential))
        lowered_variants.clear()   # protocols are known only now
        fixed_schedule = (schedule_space.fixed_schedule()
                          if schedule_space.is_fixed else None)
        edge_multiplicity = any(
            configuration[4] in (PUSH_DEPENDENCE, MAILBOX_DEPENDENCE)
            for configuration in schedule_space.configurations())
        incoming_positions = any(
            configuration[4] == MAILBOX_DEPENDENCE
            for configuration in schedule_space.configurations())
        inspector_mode = (execution_mode if fixed_schedule is not None
                          else SYNC_FREE)
        inspector_options = dict(
            validate_endpoints=validate_endpoints,
            execution_mode=inspector_mode,
            edge_multiplicity=edge_multiplicity)
        dag_source = generate_dag_source(dag_plan, **inspector_options)
        if verbose:
            print(dag_source)
        dag_builder = compile_dag_builder(
            dag_plan, device=device_layer, **inspector_options)
        rule_arrays = []
        for rule in dag_plan.edge_rules:
            for name in (getattr(rule, "pointer_array", None),
                         getattr(rule, "index_array", None)):
                if name is None:
                    continue
                if name not in rule_arrays:
                    rule_arrays.append(name)
        fingerprint_names = rule_arrays + [
            name for name in pointer_array_names(function_props)
            + structural_argument_names(structural_lookups)
            if name not in rule_arrays]
        flops_per_iteration = count_inner_loop_flops(
            function_ast, loop, thread_loop)
        thread_loop_node = None
        if thread_loop is not None:
            thread_loop_node = next(
                (node for node in ast.walk(loop_node)
                 if isinstance(node, ast.For)
                 and isinstance(node.target, ast.Name)
                 and node.target.id == thread_loop), None)
        trip_counter = {"probe": None}
        schedule_plans = {}

        def bind_arguments(args, call_kwargs):
            bound = signature.bind(*args, **call_kwargs)
            bound.apply_defaults()
            return bound.arguments

        def dag_values_for(argument_values):
            values = dict(argument_values)
            values.update(evaluate_host_prelude(
                host_lowering, values, function.__globals__,
                skip=tuple(host_lowering.zero_initialised)))
            return values

        def run_inspector(dag_values):
            return dag_builder(*[dag_values[name]
                                 for name in dag_argument_names])

        def build_dag(*args, **call_kwargs):
            return run_inspector(
                dag_values_for(bind_arguments(args, call_kwargs)))[:2]

        def trip_counts(dag_values):
            if thread_loop is None:
                return None
            fast = segment_trip_counts(thread_loop_node, loop, dag_values)
            if fast is not None:
                return fast
            if trip_counter["probe"] is None:
                trip_counter["probe"] = compile_thread_trip_counter(
                    function_ast, thread_loop, function.__globals__,
                    block_iterator=loop)
            host_values = {
                name: (value.copy_to_host()
                       if hasattr(value, "copy_to_host") else value)
                for name, value in dag_values.items()}
            return measure_thread_trip_counts(
                trip_counter["probe"], host_values, argument_names,
                sample_limit=TRIP_PROBE_SAMPLE)

        def advise(dag, band_walker):
            """The scheduler's word on a plan that belongs on the host, as
            one warning when the plan is made and as ``plan.advice``."""
            advice = sequential_advice(dag, band_walker)
            if advice is not None and kwargs.get("advice", True):
                import warnings
                warnings.warn(f"@parallel({function.__name__}): {advice}.",
                              SchedulerAdvice, stacklevel=4)
            return advice

        def create_schedule_plan(dag_values):
            device = get_device()
            # structure arrays go to HBM once per plan and stay there
            resident = {}
            for name in fingerprint_names:
                value = dag_values.get(name)
                if isinstance(value, (list, tuple)):
                    value = np.asarray(value)
                if isinstance(value, np.ndarray):
                    resident[name] = device.to_device(
                        np.ascontiguousarray(value, dtype=np.int32)
                        if np.issubdtype(value.dtype, np.integer) else value)
            device_values = dict(dag_values)
            device_values.update(resident)
            lookup_values = materialize_structural_lookups(
                structural_lookups, device_values, device)
            dag = build_device_dag(dag_plan, device_values, device,
                                   levels=True, incoming=incoming_positions)
            if fixed_schedule is not None:
                schedule = fixed_schedule
                features = None
            else:
                features = extract_workload_features(
                    dag.n, dag.levels, dag_values,
                    function_props=function_props,
                    flops_per_iteration=flops_per_iteration,
                    thread_trip_counts=trip_counts(dag_values),
                    edges=dag.edges)
                schedule = scheduler.schedule(features, schedule_space)
            # (a walker asked for by name goes before the other's automatic
            # choice)
            walker = (None if (level_option is True or sweep_option is True)
                      and walker_option != True
                      else walker_for(dag, schedule))
            if walker is not None:
                walker_dag = dag
                if not incoming_positions:
                    # (a pull-shaped loop: the walker reads the rows through
                    # the incoming listing, which this DAG was built without)
                    walker_dag = build_device_dag(
                        dag_plan, device_values, device, levels=True,
                        incoming=True)
                # the walker's table has one cell per (source, destination): a
                # structure that stores two entries for the same pair keeps
                # the executors that take every entry
                listed = walker_dag.array("in_src").shape[0]
                if listed != walker_dag.edges:
                    if walker_option is True:
                        raise ValueError(
                            "band_walker=True: the structure stores "
                            f"{listed - walker_dag.edges} entries beside "
                            "another entry of the same pair of iterations, "
                            "which the walker's table has no cell for.")
                    walker = None
                else:
                    dag = walker_dag
            if walker is not None:
                schedule, lowering = walker
                execution_data = execution_data_from_device_dag(
                    dag, schedule.execution_mode, lowering.warp_mapped,
                    band_width=band_width, mailbox=True, tile_rows=None,
                    record_lanes=None)
                plan = SchedulePlan(
                    schedule=schedule,
                    execution_data=attach_auxiliary_values(
                        execution_data, lookup_values),
                    features=features, dag=dag, tile_rows=None,
                    single_chunk=False, task_records=False,
                    band_walker=True, advice=advise(dag, True))
                plan_state[id(plan)] = {"resident": resident, "workspace": {}}
                return plan
            sweep = sweep_for(
                dag, schedule, lambda: build_device_dag(
                    dag_plan, device_values, device, levels=True,
                    incoming=True))
            if sweep is not None:
                schedule, lowering, dag, shape = sweep
                execution_data = execution_data_from_device_dag(
                    dag, schedule.execution_mode, lowering.warp_mapped,
                    band_width=band_width, mailbox=True, tile_rows=None,
                    record_lanes=None)
                plan = SchedulePlan(
                    schedule=schedule,
                    execution_data=attach_auxiliary_values(
                        execution_data, lookup_values),
                    features=features, dag=dag, tile_rows=None,
                    single_chunk=False, task_records=False,
                    grid_sweep=shape)
                plan_state[id(plan)] = {"resident": resident, "workspace": {}}
                return plan
            level = level_walker_for(
                dag, schedule, lambda: build_device_dag(
                    dag_plan, device_values, device, levels=True,
                    incoming=True))
            if level is not None:
                schedule, lowering, dag, tables, entries = level
                execution_data = execution_data_from_device_dag(
                    dag, schedule.execution_mode, lowering.warp_mapped,
                    band_width=band_width, mailbox=True, tile_rows=None,
                    record_lanes=None)
                plan = SchedulePlan(
                    schedule=schedule,
                    execution_data=attach_auxiliary_values(
                        execution_data, {**lookup_values, **tables}),
                    features=features, dag=dag, tile_rows=None,
                    single_chunk=False, task_records=False,
                    level_walker=entries)
                plan_state[id(plan)] = {"resident": resident, "workspace": {}}
                return plan
            schedule, tile_rows = tiles_for(dag, schedule, device_values)
            lowering = lower_variant(schedule.lowering_key, tile_rows)
            # the record arrays are indexed with 32 bits
            records = (not lowering.task_record_lanes
                       or dag.n * lowering.task_record_lanes < 2 ** 31)
            if not records:
                lowering = lower_variant(schedule.lowering_key, tile_rows,
                                         task_records=False)
            execution_data, tile_boxes = None, boxes_for(dag, schedule,
                                                         tile_rows)
            if (tile_boxes is not None and tile_option == "auto"
                    and kwargs.get("threads_per_block") is None
                    and schedule.threads_per_block == TILE_THREADS_PER_BLOCK):
                wider = replace(schedule,
                                threads_per_block=TILE_BOX_THREADS_PER_BLOCK)
                if boxes_for(dag, wider, tile_rows) == tile_boxes:
                    schedule = wider
                    lowering = lower_variant(schedule.lowering_key, tile_rows)
            if tile_boxes is not None:
                # a box order that is not topological, or a task with more
                # incoming edges than its record holds: tiles of consecutive
                # ids instead
                points = int(np.prod(tile_boxes[1]))
                try:
                    execution_data = execution_data_from_device_dag(
                        dag, schedule.execution_mode, lowering.warp_mapped,
                        band_width=band_width, mailbox=True, tile_rows=points,
                        record_lanes=lowering.task_record_lanes,
                        tile_boxes=tile_boxes)
                except hip_runtime.HIPRuntimeError:
                    execution_data = None
                if execution_data is None or dag.record_overflow:
                    execution_data = tile_boxes = None
                else:
                    tile_rows = points
                    lowering = lower_variant(schedule.lowering_key, points,
                                             True, True, True)
            if execution_data is None:
                execution_data = execution_data_from_device_dag(
                    dag, schedule.execution_mode, lowering.warp_mapped,
                    pushed=lowering.dependence_protocol == PUSH_DEPENDENCE,
                    band_width=band_width,
                    mailbox=lowering.dependence_protocol == MAILBOX_DEPENDENCE,
                    tile_rows=lowering.tile_rows,
                    record_lanes=lowering.task_record_lanes,
                    level_positions=lowering.level_records)
            segment_registers, structure_tables = (
                registers_for(schedule, tile_rows, device_values, lookup_values,
                              dag.n)
                if tile_boxes is None else (0, {}))
            plan = SchedulePlan(
                schedule=schedule,
                execution_data=attach_auxiliary_values(
                    execution_data, {**lookup_values, **structure_tables}),
                features=features, dag=dag, tile_rows=tile_rows,
                # every task's incoming edges fit its record: the executor
                # variant without the code for further chunks
                single_chunk=bool(lowering.task_record_lanes)
                and getattr(dag, "record_overflow", 1) == 0,
                task_records=records, tile_boxes=tile_boxes,
                segment_registers=segment_registers,
                advice=advise(dag, False))
            plan_state[id(plan)] = {"resident": resident, "workspace": {}}
            return plan

        plan_state = {}

        def plan_for(argument_values):
            dag_values = dag_values_for(argument_values)
            fingerprint = inspection_fingerprint(
                dag_values, fingerprint_names,
                device_layer if device_layer is not None else None)
            plan = schedule_plans.get(fingerprint)
            if plan is None:
                plan = create_schedule_plan(dag_values)
                if len(schedule_plans) >= SCHEDULE_CACHE_SIZE:
                    evicted = schedule_plans.pop(next(iter(schedule_plans)))
                    plan_state.pop(id(evicted), None)
                schedule_plans[fingerprint] = plan
            return plan

        def schedule_plan(*args, **call_kwargs):
            return plan_for(bind_arguments(args, call_kwargs))

        def schedule_call(*args, **call_kwargs):
            return schedule_plan(*args, **call_kwargs).schedule

        def build_execution_data(*args, **call_kwargs):
            return schedule_plan(*args, **call_kwargs).execution_data

        def publish_variant(schedule, lowering, compiled):
            if (wrapper.current_schedule == schedule
                    and wrapper.__dict__.get("hip_lowering") is lowering):
                return
            wrapper.current_schedule = schedule
            wrapper.__dict__.update(_variant_attributes(lowering, compiled))

        def resolve_call(args, call_kwargs):
            argument_values = bind_arguments(args, call_kwargs)
            plan = plan_for(argument_values)
            lowering, compiled = compile_variant(plan.schedule.lowering_key,
                                                 plan.tile_rows,
                                                 plan.single_chunk,
                                                 plan.task_records,
                                                 plan.tile_boxes is not None,
                                                 plan.segment_registers,
                                                 plan.band_walker,
                                                 plan.level_walker,
                                                 plan.grid_sweep)
            publish_variant(plan.schedule, lowering, compiled)
            state = plan_state[id(plan)]
            values = dict(argument_values)
            values.update(state["resident"])
            prepared = prepare_hip_arguments(
                lowering=lowering, argument_values=values,
                execution_data=plan.execution_data,
                function_globals=function.__globals__,
                hip_module=get_device(), compiled_module=compiled,
                workspace=state["workspace"])
            return lowering, compiled, prepared

        def prepare_hip_call(*args, **call_kwargs):
            return resolve_call(args, call_kwargs)[2]

        def bind(*args, **call_kwargs):
            """Resolve one call without running it: returns an object with
            ``launch()`` (enqueue, no sync), ``synchronize()``, ``result()``
            (download what the function returns) for callers that keep their
            data in HBM between solves."""
            lowering, compiled, prepared = resolve_call(args, call_kwargs)
            return BoundCall(lowering, compiled, prepared,
                             function.__globals__)

        @functools.wraps(function)
        def wrapper(*args, **call_kwargs):
            lowering, compiled, prepared = resolve_call(args, call_kwargs)
            return execute_hip_call(
                compiled_module=compiled, lowering=lowering,
                prepared_arguments=prepared,
                function_globals=function.__globals__)

        wrapper.original_function = function
        wrapper.build_dag = build_dag
        wrapper.build_execution_data = build_execution_data
        wrapper.prepare_hip_arguments = prepare_hip_call
        wrapper.prepare_cuda_arguments = prepare_hip_call
        wrapper.bind = bind
        wrapper.schedule_plan = schedule_plan
        wrapper.schedule_call = schedule_call
        wrapper.schedule_space = schedule_space
        wrapper.scheduler = scheduler
        wrapper.dag_plan = dag_plan
        wrapper.dag_source = dag_source
        wrapper.execution_mode = execution_mode
        wrapper.dependence_analysis = dependence_analysis
        wrapper.structural_lookups = structural_lookups
        wrapper.reduction_statements = dependence_analysis.atomic_statements
        wrapper.current_schedule = None
        wrapper.lower_variant = lower_variant
        wrapper.__dict__.update(dict.fromkeys(VARIANT_ATTRIBUTES))
        if fixed_schedule is not None:
            # an explicit tile size is known now; the automatic choice only
            # once a structure has been inspected
            rows = (tile_option if isinstance(tile_option, int)
                    and tile_option and band_width == 1 else None)
            if rows and lower_variant(fixed_schedule.lowering_key,
                                      rows).tile_rows is None:
                rows = None
            publish_variant(fixed_schedule,
                            *compile_variant(fixed_schedule.lowering_key, rows))
        return wrapper
    return decorator


class BoundCall:
    """One resolved call whose operands stay on the device."""

    def __init__(self, lowering, compiled, prepared, function_globals):
        self.lowering = lowering
        self.compiled = compiled
        self.prepared = prepared
        self.function_globals = function_globals

    @property
    def device(self):
        return self.prepared.device

    def launch(self, use_graph=True):
        launch_hip_call(self.compiled, self.lowering, self.prepared, use_graph)

    def update_values(self):
        """Tell the call that the contents of the matrix arrays have changed
        in place since it was bound (executors that keep a copy of them in
        their own layout -- the grid sweep, the level launches over operands
        in level order -- lay it out again; the arrays named in
        ``lowering.stage_static_arrays``).  Everything else, the
        right-hand side included, is read at every launch."""
        if getattr(self.lowering, "restage_launcher_name", None):
            hip_runtime.stage_static_values(
                self.compiled, self.lowering, self.prepared.values,
                self.prepared.module, self.prepared.device)

    def synchronize(self):
        self.prepared.device.synchronize()
        hip_runtime.check_executor_status(self.lowering, self.prepared)

    def device_value(self, name):
        return self.prepared.values[name]

    def result(self):
        self.synchronize()
        values = dict(self.prepared.host_values)
        for name in hip_runtime._returned_names(self.lowering.host_epilogue):
            if name in self.prepared.values:
                values[name] = self.prepared.copy_to_host(name)
        values.update(self.prepared.copy_lifted_variables_to_host())
        return hip_runtime._evaluate_host_epilogue(
            self.lowering, values, self.function_globals)

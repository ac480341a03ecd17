"""Lower one annotated Python loop to HIP C++ for gfx950 (MI355X).

Counterpart of the reference's Numba-CUDA lowering
(compiler/cuda_lowering.py): the block-mapped loop is removed, its iterator is
bound from a task list, an optional inner loop is distributed over the lanes
of a *task group*, cross-task updates become device-scope atomics, and the
result is wrapped in one of the executors.  Differences that come from
targeting CDNA4 rather than translating the CUDA code:

* Kernels are HIP C++ text built from hand-written executor templates and
  compiled at run time with hiprtc; the launcher is a small Python function
  that drives ``liblcdhip`` (level loops are captured into a hipGraph).
* A task is mapped to a group of ``task_lanes`` lanes, a power of two up to
  the 64-lane wavefront.  ``n_warp == 1`` in the reference means "one warp per
  task"; here it means one wavefront (64 lanes) unless the scheduler picks a
  narrower group, in which case one wavefront carries ``64 / task_lanes``
  tasks.  ``n_warp > 1`` makes ``n_warp`` wavefronts (one workgroup) cooperate.
* Sync-free executors are persistent: wavefronts fetch tasks in topological
  (level) order from a global counter and *poll* readiness inside a
  wave-uniform loop, so tasks that share a wavefront cannot deadlock each
  other and every wait is bounded by a watchdog.
* Statements outside the distributed loop are executed by every lane of the
  group (uniform control flow); their stores are issued by lane 0 and
  followed by a group-scope fence.
"""

import ast
from copy import deepcopy
import textwrap

from lcd_amd.structural_lookups import (
    match_segment_search,
    rewrite_structural_lookups,
    segmented_array_pairs,
    structural_lookup_names,
    structure_aliases,
)
from lcd_amd.hip_emitter import (
    COUNTER_DEPENDENCE,
    DEFAULT_SPIN_LIMIT,
    DEPENDENCE_PROTOCOLS,
    FLOAT,
    GATHER_ARGUMENTS,
    HIPLoweringError,
    HIPLoweringResult,
    INT,
    LEVEL_WALKER_ARGUMENTS,
    LEVEL_WALKER_LEVELS,
    LEVEL_WALKER_TASKS,
    MAILBOX_ARGUMENTS,
    MAILBOX_DEPENDENCE,
    PULL_ARGUMENTS,
    PULL_DEPENDENCE,
    PUSH_ARGUMENTS,
    PUSH_DEPENDENCE,
    RECORD_ARGUMENTS,
    STATUS_ARGUMENT,
    SYNC_FREE_ARGUMENTS,
    VALUE_PULL_ARGUMENTS,
    VALUE_WAIT_BEGIN,
    VALUE_WAIT_END,
    WAVEFRONT_ARGUMENTS,
    WAVEFRONT_SIZE,
    _Emitter,
    _Kinds,
    _MappedLoopHooks,
    _is_range_loop,
    _names_in,
    _normalize_mode,
    _normalize_reductions,
    _stored_names,
    _to_module,
)
from lcd_amd.hip_prelude import (
    _GROUP_SYNC_BLOCK,
    _GROUP_SYNC_WAVE,
    _PRELUDE,
)
from lcd_amd.hip_emitter import (  # noqa: F401  (re-exported)
    UnsupportedAtomicOperation,
    HIP_EXECUTION_MODES,
    HOST_LAUNCH_ARGUMENTS,
)
from lcd_amd.hip_protocols import ProtocolMixin
from lcd_amd.hip_sequential_pull import SequentialPullMixin
from lcd_amd.hip_task_transforms import TaskTransformMixin
from lcd_amd.hip_band_walker import BandWalkerMixin
from lcd_amd.hip_grid_sweep import (
    SWEEP_ARGUMENTS,
    SWEEP_FLOAT_ARGUMENTS,
    GridSweepMixin,
)


class HIPLowerer(ProtocolMixin, SequentialPullMixin, TaskTransformMixin,
                 BandWalkerMixin, GridSweepMixin):
    def __init__(self, loop_iterator, reductions=None, kernel_name=None,
                 execution_mode="plain", sync_free_ready_count=0,
                 wavefront_threads_per_block=128, thread_loop_iterator=None,
                 thread_unroll_factor=1, n_warp=None,
                 dependence_protocol=COUNTER_DEPENDENCE, direct_dependence=None,
                 function_props=None, structural_lookups=(), task_lanes=None,
                 chain_tasks=False, argument_kinds=None,
                 spin_limit=DEFAULT_SPIN_LIMIT, resident_waves_per_cu=None,
                 spin_sleep=1, promote_own_elements=True,
                 prefetch_node_loads=True, value_flags=True,
                 gather_messages=True, segment_cache=True, tile_rows=None,
                 stage_operands=True, task_records=True, single_chunk=False,
                 queue_node_loads=True, plain_first_polls=None,
                 publish_values=True, look_ahead=True, segment_capacity=None,
                 pipeline_fetch=True, full_fences=False,
                 dynamic_fetch=False, tile_positions=None,
                 tile_by_position=False, segment_registers=False,
                 pair_tables=True, band_walker=False, level_walker=0,
                 prepared_division=True, grid_sweep=None,
                 watchdog_seconds=None, level_records=True):
        self.tile_positions = tile_positions
        # level launches that gather: operands laid out in level order
        self.level_records_enabled = bool(level_records)
        self._level_records = None
        # entries per task record (the lanes of a task; four for the level
        # launches that give a task to one lane, see `_level_wide_lines`)
        self.record_lanes = 1
        self.watchdog_seconds = watchdog_seconds
        # (nx, ny, nz, WY, GY, GZ, SKZ): the grid sweep over this grid
        self.grid_sweep = tuple(grid_sweep) if grid_sweep else None
        self._sweep = None
        self.band_walker = bool(band_walker)
        # > 0: the level walker, with room for this many incoming entries per task
        self.level_walker = int(level_walker or 0)
        self._walker = None
        # locals the emitter adds while it writes the task (declared with the rest)
        self._extra_locals = []
        # the node load a task divides by (its reciprocal is prepared where
        # the pipelined fetch takes the load over), and whether a fetch did so
        self.prepared_division = prepared_division
        self._prepared_divisor = None
        self._prepared_division_active = False
        self.tile_by_position = tile_by_position
        self.segment_registers = segment_registers
        self.pair_tables = pair_tables
        # full_fences: agent-scope release/acquire fences of the HIP memory
        # model (L2 write-back / invalidate per hand-off) instead of the
        # wait-for-completion scheme; dynamic_fetch: the flat queue hands out
        # task batches from the global counter instead of round-robin, which
        # needs no exact residency of the grid.  Both are the conservative
        # forms to select when the machine is shared or a new part is brought
        # up; the defaults are faster.
        self.full_fences = bool(full_fences)
        self.dynamic_fetch = bool(dynamic_fetch)
        self.pipeline_fetch = pipeline_fetch
        self.look_ahead = look_ahead
        self.segment_capacity = segment_capacity
        self.queue_node_loads_enabled = queue_node_loads
        self.publish_values = publish_values
        self._published = None
        self.plain_first_polls = plain_first_polls
        # accessors of a producer's value-flagged element.  Unless the option
        # says otherwise the pull loop tries a plain load first (the value is
        # often there already and then comes from this XCD's L2: -4 % on the
        # power-law factor) and the gathered mailbox polls coherently (its
        # sources are mostly not ready yet: the extra load cost 5 % on the
        # 128^3 grid).
        self.pull_load = ("lcd_ld" if plain_first_polls is False
                          else "lcd_ld_once")
        self.poll_load = "lcd_ld_once" if plain_first_polls else "lcd_ld"
        self._queue_node_loads = []
        self._queue_load_lines = []
        self.stage_operands = stage_operands
        self.task_records = task_records
        self.single_chunk = single_chunk
        self.tile_rows = tile_rows
        self._tile = None
        self.segment_cache = segment_cache
        self._segment = None
        self.gather_messages = gather_messages
        self.value_flags = value_flags
        self._value_pull = None
        self._sequential_pull = None
        self._own_zero_arrays = set()
        self.promote_own_elements = promote_own_elements
        self.prefetch_node_loads = prefetch_node_loads
        self.resident_waves_per_cu = resident_waves_per_cu
        self.spin_sleep = spin_sleep
        self.loop_iterator = loop_iterator
        self.thread_loop_iterator = thread_loop_iterator
        self.reductions = _normalize_reductions(reductions)
        self.kernel_name = kernel_name
        self.execution_mode = _normalize_mode(execution_mode)
        self.sync_free_ready_count = sync_free_ready_count
        self.threads_per_block = wavefront_threads_per_block
        self.thread_unroll_factor = thread_unroll_factor
        self.n_warp = n_warp
        self.function_props = function_props or {}
        self.structural_lookups = tuple(structural_lookups or ())
        self.chain_tasks = chain_tasks
        self.argument_kinds = argument_kinds
        self.spin_limit = spin_limit
        if not isinstance(sync_free_ready_count, int):
            raise HIPLoweringError(
                "The sync-free readiness count must be an integer.")
        if (not isinstance(wavefront_threads_per_block, int)
                or wavefront_threads_per_block <= 0
                or wavefront_threads_per_block > 1024):
            raise HIPLoweringError(
                "The thread-block size must be an integer in [1, 1024].")
        if not isinstance(thread_unroll_factor, int) or thread_unroll_factor <= 0:
            raise HIPLoweringError(
                "The thread unroll factor must be a positive integer.")
        if thread_unroll_factor != 1 and thread_loop_iterator is None:
            raise HIPLoweringError(
                "A thread unroll factor requires a thread-mapped loop.")
        if n_warp is not None and (not isinstance(n_warp, int) or n_warp <= 0):
            raise HIPLoweringError("n_warp must be a positive integer.")
        if dependence_protocol not in DEPENDENCE_PROTOCOLS:
            raise HIPLoweringError(
                f"Unknown dependence protocol {dependence_protocol!r}.")
        tpb = self.threads_per_block
        self.block_task = (thread_loop_iterator is not None
                           and n_warp is not None and n_warp > 1)
        if self.block_task:
            if tpb != n_warp * WAVEFRONT_SIZE:
                raise HIPLoweringError(
                    f"n_warp={n_warp} maps one task to "
                    f"{n_warp * WAVEFRONT_SIZE} threads, but "
                    f"threads_per_block={tpb}.")
            self.task_lanes = tpb
        elif thread_loop_iterator is None:
            self.task_lanes = 1
        else:
            lanes = task_lanes if task_lanes is not None else min(
                WAVEFRONT_SIZE, tpb)
            if (lanes <= 0 or lanes & (lanes - 1) or lanes > WAVEFRONT_SIZE
                    or tpb % lanes):
                raise HIPLoweringError(
                    "task_lanes must be a power of two <= 64 that divides "
                    f"threads_per_block; got {lanes} with {tpb}.")
            self.task_lanes = lanes
        self.record_lanes = self.task_lanes
        if self.execution_mode != "plain" and not self.block_task and (
                tpb % WAVEFRONT_SIZE and tpb > WAVEFRONT_SIZE):
            raise HIPLoweringError(
                "threads_per_block must be a multiple of the 64-lane "
                f"wavefront; got {tpb}.")
        # "warp mapped" in the reference: one warp cooperates on one task.
        self.warp_mapped = (
            thread_loop_iterator is not None and not self.block_task
            and self.execution_mode in {"sync_free", "wavefront"})
        self.direct_dependence = direct_dependence
        required_kind = (PUSH_DEPENDENCE
                         if dependence_protocol == MAILBOX_DEPENDENCE
                         else dependence_protocol)
        # level launches with the mailbox protocol: a task gathers its
        # incoming products (no polls: its producers ran in earlier launches)
        self.level_gather = (
            dependence_protocol == MAILBOX_DEPENDENCE
            and direct_dependence is not None
            and direct_dependence.kind == PUSH_DEPENDENCE
            and self.warp_mapped and self.execution_mode == "wavefront"
            and not chain_tasks)
        # level launches of a task with a sequential producer loop (ILU0's
        # pivot loop): the task of the persistent pull executor -- own
        # segment in registers, searches in tables, structure located one
        # producer ahead -- with plain loads where that one polls (every
        # producer ran in an earlier launch)
        self.level_pull = (
            dependence_protocol == PULL_DEPENDENCE
            and direct_dependence is not None
            and direct_dependence.kind == PULL_DEPENDENCE
            and getattr(direct_dependence, "sequential", False)
            and self.warp_mapped and self.execution_mode == "wavefront"
            and not chain_tasks and self.task_lanes == 64
            and bool(segment_registers) and bool(pair_tables))
        self.dependence_protocol = (
            dependence_protocol
            if (direct_dependence is not None
                and direct_dependence.kind == required_kind
                and self.warp_mapped and self.execution_mode == "sync_free"
                and sync_free_ready_count == 0
                # the members of a chain task wait on their counters one by
                # one (compiler/cuda_lowering.py:1360-1410)
                and not chain_tasks) or self.level_gather or self.level_pull
            else COUNTER_DEPENDENCE)
        if chain_tasks:
            self.tile_rows = None
        self._mailbox = None
        self.group_sync = (_GROUP_SYNC_BLOCK if self.block_task
                           else _GROUP_SYNC_WAVE)
        self.segmented_sorted = segmented_array_pairs(self.function_props)

    # ---- helpers used by the hooks
    def group_total(self, partial):
        if self.block_task:
            return f"lcd_block_sum({partial}, _lcd_reduce)"
        if self.task_lanes == 1:
            return partial
        return f"lcd_group_sum({partial})"

    # ---- main entry
    def lower(self, code):
        module = _to_module(code)
        module = rewrite_structural_lookups(
            module, self.structural_lookups, self.function_props)
        functions = [n for n in module.body
                     if isinstance(n, (ast.FunctionDef, ast.AsyncFunctionDef))]
        if len(functions) != 1 or not isinstance(functions[0], ast.FunctionDef):
            raise HIPLoweringError(
                "HIP lowering expects exactly one synchronous function.")
        function = functions[0]
        function.decorator_list = []
        self._sweep_function_name = function.name
        top_index, target_loop, enclosing = self._target_loop(function)
        self._target_loop_cache = target_loop
        self.host_loops = enclosing
        host_loop_iterators = [loop.target.id for loop in enclosing]
        host_prelude = deepcopy(function.body[:top_index])
        host_epilogue = deepcopy(function.body[top_index + 1:])
        arguments = [a.arg for a in function.args.args]
        body = deepcopy(target_loop.body)
        body = self._lower_sorted_searches(body)

        loaded = set()
        for statement in body:
            loaded |= {n.id for n in ast.walk(statement)
                       if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load)}
        loaded |= _names_in(target_loop.iter)
        prelude_names = _stored_names(host_prelude)
        subscripted = {
            n.value.id for s in body for n in ast.walk(s)
            if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name)}
        lifted_variables = [
            name for name in prelude_names
            if name in loaded and name not in arguments and name in subscripted]
        lifted_loop_parameters = [
            name for name in prelude_names
            if name in loaded and name not in arguments
            and name not in subscripted]
        zero_initialised = self._zero_initialised(host_prelude, lifted_variables)

        lookup_names = structural_lookup_names(self.structural_lookups)
        kinds = _Kinds(function, self.function_props, lookup_names,
                       self.argument_kinds)
        for name in lifted_variables:
            kinds.arrays.setdefault(name, FLOAT)
        for name in lifted_loop_parameters:
            kinds.scalars[name] = INT
        for name in host_loop_iterators:
            kinds.scalars[name] = INT
        local_names = [
            name for name in _stored_names(body)
            if name not in arguments and name not in lifted_variables]
        kinds.infer_locals(body)
        self._kinds = kinds
        lowered_ids = set()
        written_arrays = self._written_arrays(body)
        self._all_written = set(written_arrays)
        if self.dependence_protocol == MAILBOX_DEPENDENCE:
            self._mailbox = self._mailbox_plan(body)
            if self._mailbox is None:
                self.dependence_protocol = (COUNTER_DEPENDENCE
                                            if self.level_gather
                                            else PUSH_DEPENDENCE)
                self.level_gather = False
        self._fully_rewritten = self._fully_rewritten_arrays(
            body, target_loop, zero_initialised)
        sequential = (self.direct_dependence is not None
                      and getattr(self.direct_dependence, "sequential", False))
        if self.dependence_protocol == PULL_DEPENDENCE and sequential:
            self._sequential_pull = self._sequential_pull_plan(body)
            if self._sequential_pull is None:
                self.dependence_protocol = COUNTER_DEPENDENCE
        elif (self.dependence_protocol == PULL_DEPENDENCE and self.value_flags
                and self.execution_mode == "sync_free"):
            self._value_pull = self._value_pull_plan(body)
        if ((self.band_walker or self.level_walker or self.grid_sweep)
                and self._value_pull is not None
                and self.dependence_protocol == PULL_DEPENDENCE):
            # the pull-shaped solve in the terms of the gathered mailbox: the
            # walker serves both
            self._mailbox = self._band_walker_pull_box(body)
            if self._mailbox is not None:
                self.dependence_protocol = MAILBOX_DEPENDENCE
                self._value_pull = None
        if self._mailbox is not None and (
                self._mailbox["array"] in self._fully_rewritten):
            self._own_zero_arrays.add(self._mailbox["array"])
            if (self.gather_messages and self.value_flags
                    and self._mailbox["gather"] is None):
                self._mailbox["gather"] = self._gather_plan(
                    self._mailbox, arguments, lifted_loop_parameters)
        if self.band_walker or self.level_walker or self.grid_sweep:
            self._walker = self._band_walker_plan(target_loop)
            if self._walker is not None and self.grid_sweep:
                self._walker.update(kind="sweep")
                for name in SWEEP_ARGUMENTS:
                    kinds.arrays[name] = (FLOAT if name in SWEEP_FLOAT_ARGUMENTS
                                          else INT)
            elif self._walker is not None and self.level_walker:
                self._walker.update(kind="level", entries=self.level_walker)
                for name in LEVEL_WALKER_ARGUMENTS:
                    kinds.arrays[name] = INT
                kinds.scalars[LEVEL_WALKER_LEVELS] = INT
            if self._walker is None:
                raise HIPLoweringError(
                    "The band walker needs the persistent executor's gathered "
                    "mailbox form: a loop over range(count) whose tasks add "
                    "`operand[j] * X[i]` to later elements of a zero-"
                    "initialised X, and at least two wavefronts per workgroup.")
            gather = self._mailbox["gather"]
            for name in gather["staged"].values():
                kinds.arrays.pop(name, None)
            gather["staged"] = {}
            gather["needs_position"] = True
            self.tile_rows = None
            self.task_records = False
            self.segment_cache = False
            self.queue_node_loads_enabled = False
        # arrays other tasks of the same launch write go through coherent
        # accessors: always in the persistent executor, and in a level launch
        # when a chain task reads what its earlier members wrote
        coherent = (set(written_arrays)
                    if self.execution_mode == "sync_free" or self.chain_tasks
                    else set())
        if self._mailbox is not None and self._mailbox["gather"] is None:
            # only a task itself touches its element of the reduced array
            coherent.discard(self._mailbox["array"])
        if self.segment_cache and not self.block_task:
            self._segment = self._segment_plan(body, arguments)
        if (self.publish_values and self._sequential_pull is not None
                and self._segment is not None and self.task_lanes == 64
                and set(self._all_written) == {self._segment["array"]}
                and kinds.arrays.get(self._segment["array"]) == FLOAT):
            # One row per wavefront, every write inside the task's own
            # segment: the final values are the messages.  They go to a
            # buffer of the array's size that starts as the empty marker, a
            # read of another task's element polls it there, and `done`, the
            # release fence ahead of it and the acquire behind the wait all
            # disappear from the chain between two levels.
            self._published = {"array": self._segment["array"],
                               "buffer": "_lcd_pub",
                               # level launches: the array itself holds the
                               # producers' final values, no buffer beside it
                               "plain": self.level_pull}
            if not self.level_pull:
                kinds.arrays["_lcd_pub"] = FLOAT
        if self.level_gather:
            if self._mailbox["gather"] is None:
                # the loop does not fit the gathered form: atomics as before
                self._mailbox = None
                self.dependence_protocol = COUNTER_DEPENDENCE
                self.level_gather = False
            else:
                gather = self._mailbox["gather"]
                for name in gather["staged"].values():
                    kinds.arrays.pop(name, None)
                gather["staged"] = {}
                gather["needs_position"] = True
                # the first incoming entries of a task from its record in
                # level order: one dependent load less in front of every task
                gather["records"] = bool(self.task_records)
                # (a plain load: nothing here is still being written)
                self.poll_load = "lcd_ld_once"
                if gather["records"] and self.level_records_enabled:
                    self._level_records = self._level_records_plan(body)
        self._segment_registers_plan(body)
        self._structure_tables = self._pair_table_plan(body)
        if self.level_pull and not (
                self._published is not None and self._segment is not None
                and self._segment.get("registers")
                and self._segment.get("foreign")):
            raise HIPLoweringError(
                "Level launches of a sequential producer loop with the pull "
                "protocol need a task whose own segment fits the registers "
                "of a wavefront and whose reads of other segments all go "
                "through the inspector's tables.")
        if self.tile_rows:
            self._tile = self._tile_plan(target_loop)
        if (self.task_records and self._mailbox is not None
                and self._mailbox["gather"] is not None
                and not self.level_gather):
            # the first incoming edges of every task sit in fixed-size
            # records in task order, so everything a wavefront needs to start
            # polling is fetched with loads whose addresses depend on the
            # task's queue position alone; operands are read through the
            # recorded positions (no per-launch staging kernel).  128^3 grid:
            # 0.475 -> 0.395 ms tiled, 0.685 -> 0.567 ms with the flat queue.
            gather = self._mailbox["gather"]
            for name in gather["staged"].values():
                kinds.arrays.pop(name, None)
            gather["staged"] = {}
            gather["needs_position"] = True
            gather["records"] = True
        if self.tile_by_position:
            self._tile_by_position_plan()
        emitter = _Emitter(kinds, self.reductions, lowered_ids,
                           coherent_arrays=coherent)
        emitter.segment = self._segment
        emitter.published = self._published
        # (the tile of a published pull mirrors the publication buffer, not
        # the array itself: its accesses go through the segment accessors)
        emitter.tile = (None if self._tile and self._tile.get("published")
                        else self._tile)
        emitter.mailbox = self._mailbox
        emitter.lowerer = self
        self._emitter = emitter

        user_arguments = list(arguments)
        for name in lifted_variables + lifted_loop_parameters:
            if name not in user_arguments:
                user_arguments.append(name)
        for name in host_loop_iterators:
            if name not in user_arguments and name in loaded:
                user_arguments.append(name)
        for name in lookup_names:
            if name not in user_arguments:
                user_arguments.append(name)
        for entry in self._structure_tables:
            user_arguments.append(entry[1])
            if entry[0] == "pair":
                user_arguments.append("_lcd_pair_base")
        if self._walker is not None and self._walker["kind"] == "level":
            user_arguments += [*LEVEL_WALKER_ARGUMENTS, LEVEL_WALKER_LEVELS]
        if self._walker is not None and self._walker["kind"] == "sweep":
            user_arguments += list(SWEEP_ARGUMENTS)
        if (self.thread_loop_iterator is not None
                and self.dependence_protocol != COUNTER_DEPENDENCE
                and self._sequential_pull is None):
            nested = self._find_mapped_loop(body)
            if nested not in body:
                # hooks describe task-level edges; a nested work-sharing loop
                # would change their multiplicity
                self.dependence_protocol = COUNTER_DEPENDENCE
        executor_arguments = self._executor_arguments()
        kernel_arguments = user_arguments + [
            name for name in executor_arguments if name not in user_arguments]

        self._lifted_parameters = list(lifted_loop_parameters)
        task_body = self._task_body(body, emitter, local_names, target_loop,
                                    arguments)
        # structure arrays the tasks read in queue order (found while the
        # node loads were hoisted) come last
        for name, _, _ in self._queue_node_loads:
            executor_arguments.append(name)
            kernel_arguments.append(name)
        if self._level_records is not None:
            # (the node values in level order were found with the node loads)
            for _, staged, _, _ in self._level_records["values"]:
                executor_arguments.append(staged)
                kernel_arguments.append(staged)
        missing = ({sid for sid, _ in self.reductions.values()} - lowered_ids)
        if missing:
            raise HIPLoweringError(
                "Reduction statements were not found in the selected loop: "
                + ", ".join(sorted(missing)))

        function_name = function.name
        self._sweep_function_name = function_name
        kernel_name = self.kernel_name or function_name + "_hip_kernel"
        launcher_name = function_name + "_hip_launch"
        reset_name = None
        array_arguments = {
            name: kinds.arrays[name] for name in kernel_arguments
            if name in kinds.arrays}
        scalar_arguments = {
            name: kinds.scalars.get(name, INT) for name in kernel_arguments
            if name not in array_arguments}
        for name in ("band_start", "band_end", "task_count"):
            if name in scalar_arguments:
                scalar_arguments[name] = INT

        kernel_text = self._kernel_text(
            kernel_name, kernel_arguments, array_arguments, scalar_arguments,
            written_arrays, task_body, local_names, target_loop)
        reset_text = ""
        if self.execution_mode == "sync_free":
            reset_name = function_name + "_hip_reset"
            reset_text = self._reset_kernel_text(reset_name)
        stage_name, stage_arguments = None, ()
        if (self._mailbox is not None and self._mailbox["gather"] is not None
                and self._mailbox["gather"]["staged"]):
            stage_name = function_name + "_hip_stage"
            stage_text, stage_arguments = self._stage_kernel_text(stage_name)
            reset_text += stage_text
        self._stage = (stage_name, stage_arguments)
        source = self._module_text(
            array_arguments, scalar_arguments, reset_text, kernel_text)
        launcher_source, launcher_arguments = self._launcher_text(
            launcher_name, kernel_name, reset_name, kernel_arguments)
        return HIPLoweringResult(
            source=source,
            kernel_source=kernel_text,
            launcher_source=launcher_source,
            launcher_ast=ast.parse(launcher_source),
            kernel_name=kernel_name,
            launcher_name=launcher_name,
            reset_kernel_name=reset_name,
            stage_kernel_name=stage_name,
            stage_kernel_arguments=tuple(stage_arguments),
            kernel_arguments=kernel_arguments,
            launcher_arguments=launcher_arguments,
            lifted_variables=lifted_variables,
            lifted_loop_parameters=lifted_loop_parameters,
            host_prelude=host_prelude,
            host_epilogue=host_epilogue,
            atomic_statement_ids=lowered_ids,
            execution_mode=self.execution_mode,
            auxiliary_arguments=[*lookup_names, *executor_arguments],
            thread_loop_iterator=self.thread_loop_iterator,
            thread_unroll_factor=self.thread_unroll_factor,
            host_loop_iterators=tuple(host_loop_iterators),
            n_warp=self.n_warp,
            warp_mapped=self.warp_mapped,
            dependence_protocol=self.dependence_protocol,
            task_lanes=self.task_lanes,
            threads_per_block=self.threads_per_block,
            tasks_per_block=max(1, self.threads_per_block // self.task_lanes),
            array_arguments=array_arguments,
            scalar_arguments=scalar_arguments,
            written_arrays=tuple(sorted(written_arrays)),
            zero_initialised=zero_initialised,
            persistent=self.execution_mode == "sync_free",
            function_name=function_name,
            mailbox_index_array=(self._mailbox["index_array"]
                                 if self._mailbox else None),
            tile_rows=self._tile["rows"] if self._tile else None,
            tile_by_position=bool(self._tile
                                  and self._tile.get("by_position")),
            band_walker=bool(self._walker
                             and self._walker["kind"] == "band"),
            level_walker=(self.level_walker if self._walker
                          and self._walker["kind"] == "level" else 0),
            grid_sweep=(dict(self._sweep["geometry"]) if self._sweep else None),
            stage_kernels=(tuple(self._sweep["kernels"]) if self._sweep
                           else tuple(self._level_records["kernels"])
                           if self._level_records else ()),
            sweep_dynamic=bool(self._sweep and self._sweep["dynamic_kernel"]),
            stage_static_arrays=(tuple(self._sweep["static_arrays"])
                                 if self._sweep
                                 else tuple(self._level_records["static_arrays"])
                                 if self._level_records else ()),
            restage_launcher_name=(function_name + "_hip_sweep_restage"
                                   if self._sweep
                                   else function_name + "_hip_level_restage"
                                   if self._level_records else None),
            level_records=self._level_records is not None,
            segment_pointer=(self._segment["pointer"]
                             if self._segment else None),
            segment_registers=bool(self._segment
                                   and self._segment.get("registers")),
            structure_tables=tuple(self._structure_tables),
            spin_limit=self.spin_limit,
            watchdog_seconds=self.watchdog_seconds,
            queue_node_loads=tuple(self._queue_node_loads),
            published_array=(self._published["array"]
                             if self._published else None),
            task_record_lanes=(
                self.record_lanes if self._mailbox
                and self._mailbox["gather"]
                and self._mailbox["gather"].get("records") else None),
            value_flag_array=(
                self._value_pull["array"] if self._value_pull
                else self._mailbox["array"]
                if self._mailbox and self._mailbox["gather"] else None),
            executor_initialised=tuple(sorted(
                self._own_zero_arrays
                | ({self._value_pull["array"]} if self._value_pull else set()))),
        )

    # ---- structure discovery
    def _target_loop(self, function):
        matches = []

        def search(statements, enclosing, top_index):
            for index, statement in enumerate(statements):
                top = index if top_index is None else top_index
                if not isinstance(statement, ast.For):
                    continue
                if (isinstance(statement.target, ast.Name)
                        and statement.target.id == self.loop_iterator):
                    matches.append((top, statement, tuple(enclosing)))
                    continue
                search(statement.body, enclosing + [statement], top)

        search(function.body, [], None)
        if len(matches) != 1:
            raise HIPLoweringError(
                f"Expected exactly one top-level loop over "
                f"{self.loop_iterator!r}; found {len(matches)}.")
        top_index, loop, enclosing = matches[0]
        if not _is_range_loop(loop):
            raise HIPLoweringError(
                "The block-mapped loop must iterate over range(...).")
        for outer, inner in zip(enclosing, list(enclosing[1:]) + [loop]):
            if not _is_range_loop(outer) or outer.body != [inner]:
                raise HIPLoweringError(
                    "Loops enclosing the block-mapped loop may contain only "
                    "the next loop.")
        return top_index, loop, enclosing

    def _zero_initialised(self, host_prelude, lifted_variables):
        """``x = np.zeros(expr)`` in the prelude: allocate and zero on the
        device instead of building the array on the host."""
        found = {}
        for statement in host_prelude:
            if not (isinstance(statement, ast.Assign)
                    and len(statement.targets) == 1
                    and isinstance(statement.targets[0], ast.Name)
                    and statement.targets[0].id in lifted_variables):
                continue
            call = statement.value
            if (isinstance(call, ast.Call)
                    and isinstance(call.func, ast.Attribute)
                    and call.func.attr == "zeros"
                    and isinstance(call.func.value, ast.Name)
                    and call.func.value.id in ("np", "numpy")
                    and len(call.args) == 1 and not call.keywords):
                found[statement.targets[0].id] = ast.unparse(call.args[0])
        return found

    def _written_arrays(self, body):
        written = set()
        for statement in body:
            for node in ast.walk(statement):
                targets = []
                if isinstance(node, ast.Assign):
                    targets = node.targets
                elif isinstance(node, ast.AugAssign):
                    targets = [node.target]
                for target in targets:
                    if isinstance(target, ast.Subscript) and isinstance(
                            target.value, ast.Name):
                        written.add(target.value.id)
        return written

    def _lower_sorted_searches(self, body):
        """Equality searches over a sorted segment become a lower-bound
        search (the reference does this for nested thread-mapped loops,
        compiler/cuda_lowering.py:1640-1756)."""
        if not self.segmented_sorted:
            return body
        pairs = self.segmented_sorted
        aliases = structure_aliases(ast.Module(body=body, type_ignores=[]))

        class Searches(ast.NodeTransformer):
            def visit_For(self, node):
                node = self.generic_visit(node)
                match = match_segment_search(node, pairs, aliases)
                if match is None:
                    return node
                lower, upper = node.iter.args
                find = ast.Assign(
                    targets=[ast.Name(id=match.iterator, ctx=ast.Store())],
                    value=ast.Call(
                        func=ast.Name(id="_lcd_sorted_find", ctx=ast.Load()),
                        args=[ast.Name(id=match.index_array, ctx=ast.Load()),
                              deepcopy(lower), deepcopy(upper),
                              deepcopy(match.needle)],
                        keywords=[]))
                found = ast.If(
                    test=ast.Compare(
                        left=ast.Name(id=match.iterator, ctx=ast.Load()),
                        ops=[ast.GtE()], comparators=[ast.Constant(value=0)]),
                    body=[deepcopy(s) for s in match.matched_body]
                    or [ast.Pass()],
                    orelse=[])
                return [ast.copy_location(find, node),
                        ast.copy_location(found, node)]

        wrapper = ast.Module(body=body, type_ignores=[])
        return ast.fix_missing_locations(Searches().visit(wrapper)).body

    def _executor_arguments(self):
        if self.execution_mode == "sync_free":
            if self.dependence_protocol == PUSH_DEPENDENCE:
                names = list(PUSH_ARGUMENTS)
            elif (self.dependence_protocol == PULL_DEPENDENCE
                  and self._value_pull is not None):
                names = list(VALUE_PULL_ARGUMENTS)
            elif self.dependence_protocol == PULL_DEPENDENCE:
                names = ["_lcd_pub" if name == "done" and self._published
                         else name for name in PULL_ARGUMENTS]
            elif (self.dependence_protocol == MAILBOX_DEPENDENCE
                  and self._mailbox["gather"] is not None):
                gather = self._mailbox["gather"]
                names = [name for name in GATHER_ARGUMENTS
                         if name != "_lcd_in_pos" or gather["needs_position"]]
                names[2:2] = list(gather["staged"].values())
                if gather.get("records"):
                    position = names.index("_lcd_in_src") + 1
                    names[position:position] = list(RECORD_ARGUMENTS)
                if self._tile is not None and self._tile.get("by_position"):
                    names.append("_lcd_xq")
            elif self.dependence_protocol == MAILBOX_DEPENDENCE:
                names = list(MAILBOX_ARGUMENTS)
            else:
                names = list(SYNC_FREE_ARGUMENTS)
            return names + [STATUS_ARGUMENT]
        if self.execution_mode == "wavefront":
            return list(WAVEFRONT_ARGUMENTS) + (
                ["_lcd_in_ptr", "_lcd_in_pos", "_lcd_in_src",
                 *(RECORD_ARGUMENTS if self._mailbox["gather"].get("records")
                   else ()),
                 *([*self._level_records["operands"].values(), "_lcd_xq"]
                   if self._level_records is not None else ())]
                if self.level_gather else [])
        return []

    # ---- task body
    def _find_mapped_loop(self, body):
        if self.thread_loop_iterator is None:
            return None
        matches = [
            node for statement in body for node in ast.walk(statement)
            if isinstance(node, ast.For) and isinstance(node.target, ast.Name)
            and node.target.id == self.thread_loop_iterator]
        if len(matches) != 1:
            raise HIPLoweringError(
                "The selected thread iterator must identify exactly one inner "
                f"for loop; found {len(matches)} for "
                f"{self.thread_loop_iterator!r}.")
        if not _is_range_loop(matches[0]):
            raise HIPLoweringError(
                "The thread-mapped loop must iterate over range(...).")
        return matches[0]

    def _task_body(self, body, emitter, local_names, target_loop, arguments):
        """C++ lines of one task (indent level 0), `i` already bound."""
        gather = self._mailbox["gather"] if self._mailbox is not None else None
        if gather is not None:
            # the consumers form the products themselves: the producer's
            # distributed loop is gone
            site = self._mailbox["sites"][0]
            if self._walker is not None:
                # (the walker wants to know where the loop was: what comes
                # before it starts the task's element, what comes after ends it)
                marker = ast.Pass()
                marker._lcd_walker_split = True
                body = [marker if s is self._mailbox["mapped"] else s
                        for s in body]
            else:
                body = [s for s in body if s is not self._mailbox["mapped"]]
            location = (site.lineno, site.col_offset)
            if location in self.reductions:
                emitter.lowered_ids.add(self.reductions[location][0])
            mapped = None
        else:
            mapped = self._find_mapped_loop(body)
        hooks = None
        self._own_registers = []
        self._own_map = {}
        self._pending_sync = False
        if mapped is not None:
            hooks = _MappedLoopHooks(self, emitter, mapped)
            outer_assigned = set(local_names) - (
                {mapped.target.id} | set(_stored_names(mapped.body)))
            if not self._privatize(mapped, hooks, outer_assigned):
                raise HIPLoweringError(
                    "The thread-mapped loop writes state that cannot be "
                    "privatized safely.")
            for partial, _, _ in hooks.partials:
                self._kinds.locals[partial] = FLOAT
        prologue, epilogue = [], []
        if self.promote_own_elements:
            body, prologue, epilogue = self._promote_own_elements(
                body, mapped, hooks, arguments)
        self._hook_endpoint = self._hook_guard = None
        self._first_iteration_reload = []
        self._prefetch_lines = []
        if self._mailbox is not None:
            self._mailbox["slot"] = self._mailbox_slot_load()
        if self.prefetch_node_loads:
            body, self._prefetch_lines = self._hoist_node_loads(
                body, mapped, arguments)
        if self._walker is not None:
            body = self._band_walker_division(body)
        elif (self.prepared_division and self.execution_mode == "sync_free"
              and self.pipeline_fetch and self.prefetch_node_loads):
            body = self._prepared_division(body)
        if self._value_pull is not None:
            own = self._own_map.get(
                f"{self._value_pull['array']}[{self.loop_iterator}]")
            if own is None or mapped is None:
                raise HIPLoweringError(
                    "Value-flagged pull needs the task's own element of "
                    f"{self._value_pull['array']!r} in a register.")
            hooks.value_pull = self._value_pull
        if self._mailbox is not None:
            own = self._own_map.get(self._mailbox["own_text"])
            if own is None or (own[1] != "read"
                               and not self._mailbox.get("pulled")):
                raise HIPLoweringError(
                    "The mailbox protocol needs the task's own element of "
                    f"{self._mailbox['array']!r} in a register.")
            self._mailbox["register"] = own[0]
            # nobody else writes the own element: its initial value is loaded
            # with the other node loads, before the wait
            self._prefetch_lines = list(self._prefetch_lines) + list(prologue)
            prologue = []
        if not self.block_task:
            # (a workgroup-wide task has no lock step between the wavefronts
            # that would read the old value and the one that stores the new)
            body = self._forward_stores(body, mapped)
        if mapped is not None and self.task_lanes > 1:
            body = self._guard_stores(body, mapped)
        self._partials = hooks.partials if hooks else []
        lines = list(prologue)
        if self._segment is not None:
            stage, write_back = self._segment_lines()
            lines += stage
            epilogue = list(write_back) + list(epilogue)
        for statement in body:
            if getattr(statement, "_lcd_walker_split", False):
                self._walker["split"] = len(lines)
                continue
            lines.extend(self._emit_guarded(statement, emitter, 0, hooks))
        lines.extend(epilogue)
        if self._walker is not None:
            lines = self._band_walker_store(lines)
            if lines is None:
                raise HIPLoweringError(
                    "The band walker needs a task that ends with the one "
                    "store of its own element.")
        return lines

    def _emit_guarded(self, node, emitter, indent, hooks):
        pad = "    " * indent
        if (isinstance(node, ast.If) and getattr(node, "_lcd_store_guard", False)
                and self._segment is not None
                and self._segment.get("registers")
                and all(isinstance(child, ast.Assign)
                        and isinstance(child.targets[0], ast.Subscript)
                        and isinstance(child.targets[0].value, ast.Name)
                        and child.targets[0].value.id == self._segment["array"]
                        for child in node.body)):
            # the lane that holds the entry takes the value: every lane runs
            # the statement, nothing to fence
            return emitter.block(node.body, indent, None)
        if isinstance(node, ast.If) and getattr(node, "_lcd_store_guard", False):
            inner = emitter.block(node.body, indent + 1, None)
            self._pending_sync = False
            return [f"{pad}if (_lane == 0) {{", *inner, f"{pad}}}",
                    f"{pad}{self.group_sync}"]
        if isinstance(node, ast.If):
            lines = [f"{pad}if ({emitter.expr(node.test)}) {{"]
            for child in node.body:
                lines += self._emit_guarded(child, emitter, indent + 1, hooks)
            if node.orelse:
                lines.append(f"{pad}}} else {{")
                for child in node.orelse:
                    lines += self._emit_guarded(child, emitter, indent + 1, hooks)
            lines.append(f"{pad}}}")
            return lines
        if isinstance(node, ast.For) and not (hooks and hooks.is_mapped(node)):
            if not _is_range_loop(node):
                raise HIPLoweringError(
                    "Device loops must be `for name in range(...)`.")
            lower, upper, step = emitter.range_parts(node)
            name = node.target.id
            plan = self._sequential_pull
            if (plan is not None and indent == 0 and not plan.get("emitted")
                    and name == plan["iterator"] and step == "1"):
                return self._sequential_pull_lines(node, emitter, hooks,
                                                   lower, upper)
            if step == "1":
                head = f"{pad}for ({name} = {lower}; {name} < {upper}; ++{name}) {{"
            else:
                head = (f"{pad}for ({name} = {lower}; lcd_in_range({name}, "
                        f"{upper}, {step}); {name} += {step}) {{")
            lines = [head]
            for child in node.body:
                lines += self._emit_guarded(child, emitter, indent + 1, hooks)
            lines.append(f"{pad}}}")
            return lines
        if isinstance(node, ast.While):
            lines = [f"{pad}while ({emitter.expr(node.test)}) {{"]
            for child in node.body:
                lines += self._emit_guarded(child, emitter, indent + 1, hooks)
            lines.append(f"{pad}}}")
            return lines
        return emitter.stmt(node, indent, hooks)

    # ---- text assembly
    def _c_type(self, name, kind, is_array):
        return f"LCD_T_{name}"

    def _module_text(self, array_arguments, scalar_arguments, reset_text,
                     kernel_text):
        defines = [
            *(["#define LCD_FULL_FENCES 1"] if self.full_fences else []),
            *(["#define LCD_PREPARED_DIVISION 1"]
              if self._prepared_division_active else []),
            *(["#define LCD_DYNAMIC_FETCH 1"] if self.dynamic_fetch else []),
            "#ifndef LCD_INDEX_TYPE", "#define LCD_INDEX_TYPE int", "#endif",
            f"#define LCD_TPB {self.threads_per_block}",
            f"#define LCD_TASK_LANES {self.task_lanes}",
            f"#define LCD_RECORD_LANES {self.record_lanes}",
            f"#define LCD_GROUPS_PER_BLOCK (LCD_TPB / LCD_TASK_LANES)",
            "#ifndef LCD_SPIN_LIMIT",
            # a poll of LDS takes a tenth of a poll of memory: keep the
            # watchdog's time scale when the default limit is in use
            f"#define LCD_SPIN_LIMIT {min(self.spin_limit * (16 if self._tile is not None and self.spin_limit == DEFAULT_SPIN_LIMIT else 1), 0xFFFFF000)}",
            "#endif",
            f"#define LCD_READY_COUNT {self.sync_free_ready_count}",
            "#ifndef LCD_SPIN_SLEEP",
            f"#define LCD_SPIN_SLEEP {self.spin_sleep}", "#endif",
        ]
        if self._walker is not None and self._walker["kind"] == "level":
            defines.append(f"#define LCD_LW_TASKS {LEVEL_WALKER_TASKS}")
        if self._segment is not None:
            defines.append(f"#define LCD_SEG_CAP {self._segment['capacity']}")
        if self._tile is not None:
            defines.append(f"#define LCD_TILE_ROWS {self._tile['rows']}")
            if self._tile.get("published"):
                defines.append(
                    f"#define LCD_TILE_POS {self._tile['positions']}")
            # a poll of memory stalls the whole wavefront for a memory round
            # trip; sources outside the running tile are polled on every
            # (mask + 1)-th pass only, LDS on every pass
            defines += ["#ifndef LCD_EXTERNAL_POLL_MASK",
                        "#define LCD_EXTERNAL_POLL_MASK 0", "#endif"]
        for name, kind in array_arguments.items():
            default = "int" if kind == INT else "double"
            defines += [f"#ifndef LCD_T_{name}",
                        f"#define LCD_T_{name} {default}", "#endif"]
        for name, kind in scalar_arguments.items():
            default = "long long" if kind == INT else "double"
            if name in ("band_start", "band_end", "task_count"):
                default = "int"
            defines += [f"#ifndef LCD_T_{name}",
                        f"#define LCD_T_{name} {default}", "#endif"]
        block_sum = ""
        if self.block_task:
            block_sum = textwrap.dedent("""
            // Sum over the whole workgroup: butterfly inside each wavefront,
            // then one LDS slot per wavefront.
            __device__ __forceinline__ double lcd_block_sum(double v, double* slots) {
                for (int offset = 32; offset > 0; offset >>= 1)
                    v += __shfl_xor(v, offset, 64);
                __syncthreads();
                if ((threadIdx.x & 63) == 0) slots[threadIdx.x >> 6] = v;
                __syncthreads();
                double total = 0.0;
                for (int w = 0; w < LCD_TPB / 64; ++w) total += slots[w];
                return total;
            }
            """)
        return ("\n".join(defines) + "\n" + _PRELUDE + block_sum + reset_text
                + kernel_text)

    def _signature(self, kernel_arguments, array_arguments, scalar_arguments,
                   written_arrays):
        parts = []
        mutable_executor = {"dep_count", "task_counter", "done",
                            STATUS_ARGUMENT, "_lcd_mailbox", "_lcd_pub",
                            "_lcd_xq", *SWEEP_ARGUMENTS}
        if self._level_records is not None:
            # (written by the staging kernels, which share the signature)
            mutable_executor |= set(self._level_records["operands"].values())
            mutable_executor |= {staged for _, staged, _, _
                                 in self._level_records["values"]}
        for name in kernel_arguments:
            if name in array_arguments:
                const = (name not in written_arrays
                         and name not in mutable_executor)
                qualifier = "const " if const else ""
                restrict = " __restrict__" if const else ""
                parts.append(f"{qualifier}LCD_T_{name}*{restrict} {name}")
            else:
                parts.append(f"LCD_T_{name} {name}")
        return ",\n        ".join(parts)

    def _declarations(self, local_names, indent):
        pad = "    " * indent
        lines = []
        declared = set()
        for name in (list(local_names) + [p for p, _, _ in self._partials]
                     + list(self._own_registers) + list(self._extra_locals)):
            if name in declared or name == self.loop_iterator:
                continue
            declared.add(name)
            kind = self._kinds.locals.get(name, INT)
            if name in self._kinds.iterators:
                kind = INT
            ctype = "lcd_index_t" if kind == INT else "double"
            init = "0" if kind == INT else "0.0"
            lines.append(f"{pad}{ctype} {name} = {init};")
        return lines

    def _node_guard(self, target_loop):
        emitter = self._emitter
        lower, upper, step = emitter.range_parts(target_loop)
        tests = [f"{self.loop_iterator} < {upper}"]
        if lower != "0":
            tests.append(f"{self.loop_iterator} >= {lower}")
        return " && ".join(tests)

    def _kernel_text(self, kernel_name, kernel_arguments, array_arguments,
                     scalar_arguments, written_arrays, task_body, local_names,
                     target_loop):
        it = self.loop_iterator
        signature = self._signature(kernel_arguments, array_arguments,
                                    scalar_arguments, written_arrays)
        lines = [
            "", f'extern "C" __global__ void __launch_bounds__(LCD_TPB)',
            f"{kernel_name}(", f"        {signature})", "{",
        ]
        if self.block_task:
            lines.append("    __shared__ double _lcd_reduce[LCD_TPB / 64];")
            lines.append("    __shared__ int _lcd_task_slot;")
        lines.append("    const int _lane = threadIdx.x % LCD_TASK_LANES;")
        lines.append("    (void)_lane;")
        if self._tile is not None and self._tile.get("published"):
            lines += [
                f"    __shared__ LCD_T_{self._tile['array']} "
                "_lcd_ptile[LCD_TILE_POS];",
                "    __shared__ int _lcd_tile_slot;",
                "    lcd_index_t _lcd_tile_row0 = 0, _lcd_tile_rows = 0;",
                "    lcd_index_t _lcd_tpos0 = 0, _lcd_tlen = 0;",
            ]
        elif self._tile is not None:
            lines += [
                f"    __shared__ LCD_T_{self._tile['array']} "
                "_lcd_tile[LCD_TILE_ROWS];",
                "    __shared__ int _lcd_tile_slot;",
                "    lcd_index_t _lcd_tile_row0 = 0, _lcd_tile_rows = 0;",
            ]
        if self._published is not None and not (
                self._tile is not None and self._tile.get("published")):
            # no tile: the published accessors never look for an LDS copy
            lines += [
                f"    LCD_T_{self._published['array']}* const _lcd_ptile = nullptr;",
                "    const lcd_index_t _lcd_tpos0 = 0, _lcd_tlen = 0;",
                "    (void)_lcd_ptile; (void)_lcd_tpos0; (void)_lcd_tlen;",
            ]
        if self._segment is not None:
            array = self._segment["array"]
            lines += [
                # (no copy in LDS of a segment that lives in registers and
                # is read at run-time positions by nobody)
                *([] if self._segment.get("foreign") else [
                    f"    __shared__ LCD_T_{array} _lcd_seg_store["
                    "LCD_GROUPS_PER_BLOCK * LCD_SEG_CAP];",
                    f"    LCD_T_{array}* const _lcd_seg = &_lcd_seg_store["
                    "(threadIdx.x / LCD_TASK_LANES) * LCD_SEG_CAP];"]),
                "    lcd_index_t _lcd_seg_base = 0, _lcd_seg_limit = 0;",
                *(["    lcd_index_t _lcd_seg_own = 0;"] if self._published else []),
                *([f"    LCD_T_{array} _lcd_rseg = 0.0;",
                   "    (void)_lcd_seg_limit;"]
                  if self._segment.get("registers") else []),
                *(["    lcd_index_t _lcd_pair_row = 0;"]
                  if self._segment.get("pair_row") else []),
            ]
        lines.append(f"    lcd_index_t {it} = 0;")
        lines += self._declarations(local_names, 1)
        if self._sequential_pull is not None:
            lines.append("    bool _lcd_blocked = false;")
        guard = self._node_guard(target_loop)

        prefetch = list(self._prefetch_lines)
        self._prefetch_guard = guard

        def task(indent, body_lines=None):
            pad = "    " * indent
            out = [f"{pad}if ({guard}) {{"]
            if self._level_records is not None:
                # every node of the level order lies in the loop's range (the
                # DAG was built over it), and a test on the loaded id would
                # hold the record's loads back until the id has arrived
                out = [f"{pad}{{"]
            if self.execution_mode != "sync_free":
                out += [pad + "    " + line for line in prefetch]
            wide = (self._level_records is not None
                    and self._level_records.get("wide"))
            if wide:
                out += self._level_wide_sum_lines(indent + 1)
            elif self.level_gather:
                # the producers ran in earlier launches: their values are
                # there, the products are added in (source, position) order
                records = self._mailbox["gather"].get("records", False)
                out += [
                    # (with records the fetch sits in front of the task,
                    # beside the load of its id)
                    *([] if records else
                      [f"{pad}    const bool _pending = true;",
                       f"{pad}    int _mb_next = _lcd_in_ptr[{it}], "
                       f"_mb_end = _lcd_in_ptr[{it} + 1];",
                       *self._gather_fetch_lines(indent + 1, declare=True)]),
                    # (one turn per chunk of incoming edges; bounded, so that
                    # no content of the array can keep a launch from ending)
                    f"{pad}    const int _mb_turns = (_mb_end - _mb_next) / "
                    "LCD_TASK_LANES + 2;",
                    f"{pad}    for (int _mb_turn = 0; _mb_turn < _mb_turns; "
                    "++_mb_turn) {",
                    *self._gather_ready_lines(indent + 2),
                    f"{pad}        if (_ready) break;",
                    f"{pad}    }}",
                ]
            out += [pad + "    " + line for line in (
                task_body if body_lines is None else body_lines)]
            out.append(f"{pad}}}")
            return out

        if self._value_pull is not None or self._sequential_pull is not None:
            begin = task_body.index(VALUE_WAIT_BEGIN)
            end = task_body.index(VALUE_WAIT_END)
            self._value_segments = (task_body[:begin], task_body[begin + 1:end],
                                    task_body[end + 1:])

        def node_loop(indent, body_fn):
            pad = "    " * indent
            if self.chain_tasks:
                # a member's updates are complete and visible before the next
                # member of the chain starts
                return ([f"{pad}for (int _pos = task_ptr[_task]; "
                         f"_pos < task_ptr[_task + 1]; ++_pos) {{",
                         f"{pad}    {it} = task_nodes[_pos];",
                         *body_fn(indent + 1),
                         f"{pad}    lcd_release_fence();",
                         f"{pad}    {self.group_sync}",
                         f"{pad}}}"])
            fetch = []
            if (self._level_records is not None
                    and self._level_records.get("wide")):
                fetch = self._level_wide_fetch_lines(indent)
            elif self.level_gather and self._mailbox["gather"].get("records"):
                # the record of the task is addressed by its place in the
                # level order: its loads leave with the load of the task id
                fetch = [f"{pad}const bool _pending = true;",
                         f"{pad}int _mb_next = 0, _mb_end = 0;",
                         *self._gather_fetch_lines(indent, declare=True,
                                                   records=True)]
            return [f"{pad}{it} = task_nodes[_task];",
                    *fetch,
                    *[pad + line for line in self._queue_load_lines],
                    *body_fn(indent)]

        if self.execution_mode == "plain":
            lower, _, _ = self._emitter.range_parts(target_loop)
            lines.append("    const long long _group = "
                         "((long long)blockIdx.x * LCD_TPB + threadIdx.x) "
                         "/ LCD_TASK_LANES;")
            lines.append(f"    {it} = (lcd_index_t)(({lower}) + _group);")
            lines += task(1)
        elif self.execution_mode == "wavefront":
            lines.append("    const long long _task = (long long)band_start + "
                         "((long long)blockIdx.x * LCD_TPB + threadIdx.x) "
                         "/ LCD_TASK_LANES;")
            lines.append("    if (_task >= band_end) return;")
            lines += node_loop(1, task)
            if self._level_records is not None:
                lines.append("}")
                return (self._level_stage_kernels(
                    self._sweep_function_name, signature,
                    self._declarations(local_names, 1), guard)
                        + "\n".join(lines) + "\n")
        elif self._walker is not None:
            walker = (self._level_walker_text(task_body)
                      if self._walker["kind"] == "level"
                      else self._grid_sweep_text(task_body)
                      if self._walker["kind"] == "sweep"
                      else self._band_walker_text(task_body))
            if walker is None:
                raise HIPLoweringError(
                    "The band walker cannot stage this task's node loads."
                    if self._walker["kind"] != "sweep" else
                    "The grid sweep needs a task whose tail is arithmetic "
                    "over its node loads (+, -, *, one division by a node "
                    "load), a workgroup of (GY * GZ + GY + GZ) wavefronts "
                    "and face arrays that fit the LDS.")
            if self._walker["division"]:
                lines.append("    double _lcd_wr = 0.0;")
            lines += walker
            if self._walker["kind"] == "sweep":
                # the staging kernels share the signature and the locals
                lines.append("}")
                return (self._grid_stage_kernels(
                    self._sweep_function_name, signature,
                    self._declarations(local_names, 1))
                        + "\n".join(lines) + "\n")
        else:
            lines += self._sync_free_text(task, node_loop)
        lines.append("}")
        return "\n".join(lines) + "\n"

    def _sync_free_text(self, task, node_loop):
        """Persistent poll-loop executor.

        Wavefronts fetch ``64 / task_lanes`` consecutive tasks from the
        level-ordered queue, then loop until every one of them has run: a
        group whose dependences are satisfied executes its task inside the
        loop, the others keep polling.  Because nothing blocks inside the
        loop, tasks that share a wavefront can depend on each other.  The
        lowest unfinished task in queue order is always held by a resident
        wavefront and has all its producers finished or running, which is the
        forward-progress argument; a watchdog bounds every wait anyway.
        """
        it = self.loop_iterator
        protocol = self.dependence_protocol
        if self.chain_tasks and self.block_task:
            raise HIPLoweringError(
                "band_width > 1 (chain tasks) needs one wavefront or less per "
                "task in the persistent executor.")
        lines = ["    const int _task_count = (int)task_count;"]
        if self.block_task:
            lines += [
                "    const long long _lcd_t0 = (long long)wall_clock64();",
                "    while (true) {",
                "        if (threadIdx.x == 0)",
                "            _lcd_task_slot = atomicAdd(&task_counter[0], 1);",
                "        __syncthreads();",
                "        const int _task = _lcd_task_slot;",
                "        __syncthreads();",
                "        if (_task >= _task_count) return;",
                f"        {it} = (lcd_index_t)task_nodes[_task];",
                *["        " + line for line in self._queue_load_lines],
                f"        if ({self._prefetch_guard}) {{",
                *[f"            {line}" for line in self._prefetch_lines],
                "        }",
                "        if (threadIdx.x == 0) {",
                "            long long _spins = 0;",
                "            int _ok = 1;",
                f"            while (lcd_load_relaxed(&dep_count[{it}]) != LCD_READY_COUNT) {{",
                "                __builtin_amdgcn_s_sleep(LCD_SPIN_SLEEP);",
                "                if ((++_spins & 255) == 0 && ("
                f"lcd_gave_up(_spins, {STATUS_ARGUMENT}, _lcd_t0) || "
                f"lcd_load_relaxed(&{STATUS_ARGUMENT}[0]) != 0)) {{",
                f"                    {STATUS_ARGUMENT}[0] = 1;",
                "                    _ok = 0;",
                "                    break;",
                "                }",
                "            }",
                "            _lcd_task_slot = _ok;",
                "        }",
                "        __syncthreads();",
                "        if (!_lcd_task_slot) return;",
                "        __syncthreads();",
                "        lcd_acquire_fence();",
            ]
            lines += task(2)
            lines += [
                "        lcd_release_fence();",
                "        __syncthreads();",
                f"        for (int _e = dag_ptr[{it}] + _lane; "
                f"_e < dag_ptr[{it} + 1]; _e += LCD_TASK_LANES)",
                "            lcd_atomic_sub(&dep_count[dag_index[_e]], 1);",
                "    }",
            ]
            return lines
        tiled = self._tile is not None
        if tiled:
            # one workgroup per tile of consecutive block-iterator values,
            # its wavefronts share the tile's tasks in (level, id) order;
            # tiles are taken in increasing order, so the lowest unfinished
            # tile is always running and depends on finished tiles only.
            # With more tiles than workgroups the tiles are claimed from the
            # task counter: a workgroup that holds a tile is running by
            # construction, whereas tiles dealt out by block index wait for
            # every workgroup of the grid to be resident at once -- and the
            # occupancy query can promise more than the CUs then hold (six
            # wavefronts per workgroup do not spread evenly over four SIMDs:
            # a 256 x 256 x 128 grid stopped with a third of its tiles never
            # started).
            fetch = [
                "    const bool _lcd_claim = (long long)gridDim.x * LCD_TILE_ROWS "
                "< _task_count;",
                "    for (int _turn = 0; ; ++_turn) {",
                "    int _tile = blockIdx.x;",
                "    if (_lcd_claim) {",
                "        if (threadIdx.x == 0) _lcd_tile_slot = "
                "atomicAdd(&task_counter[0], 1);",
                "        __syncthreads();",
                "        _tile = _lcd_tile_slot;",
                "    } else if (_turn) break;",
                "    if ((long long)_tile * LCD_TILE_ROWS >= _task_count) break;",
                "    _lcd_tile_row0 = _tile * LCD_TILE_ROWS;",
                "    _lcd_tile_rows = _task_count - _lcd_tile_row0 < LCD_TILE_ROWS "
                "? _task_count - _lcd_tile_row0 : LCD_TILE_ROWS;",
                *([
                    # the tile's slice of the publication buffer
                    f"    _lcd_tpos0 = (lcd_index_t){self._tile['pointer']}"
                    "[_lcd_tile_row0];",
                    f"    _lcd_tlen = (lcd_index_t){self._tile['pointer']}"
                    "[_lcd_tile_row0 + _lcd_tile_rows] - _lcd_tpos0;",
                    "    if (_lcd_tlen > LCD_TILE_POS) _lcd_tlen = 0;",
                    "    for (int _s = threadIdx.x; _s < _lcd_tlen; _s += LCD_TPB) "
                    "_lcd_ptile[_s] = lcd_empty();",
                ] if self._tile.get("published") else [
                    "    for (int _s = threadIdx.x; _s < _lcd_tile_rows; "
                    "_s += LCD_TPB) _lcd_tile[_s] = lcd_empty();",
                ]),
                "    __syncthreads();",
                "    for (int _round = 0; ; ++_round) {",
                "        const int _local = (_round * (LCD_TPB / 64) + "
                "(int)(threadIdx.x >> 6)) * _tasks_per_wave;",
                "        if (_local >= _lcd_tile_rows) break;",
                "        const int _task = _lcd_tile_row0 + _local + "
                "(int)(threadIdx.x & 63) / LCD_TASK_LANES;",
                "        bool _pending = _task < _lcd_tile_row0 + _lcd_tile_rows;",
            ]
        else:
            fetch = [
                "    int _round = 0; (void)_round;",
                "    while (true) {",
                "#ifndef LCD_DYNAMIC_FETCH",
                "        const int _base = (_round * (int)(gridDim.x * (LCD_TPB / 64)) + "
                "(int)(blockIdx.x * (LCD_TPB / 64) + (threadIdx.x >> 6))) * _tasks_per_wave;",
                "        ++_round;",
                "#else",
                "        int _base = 0;",
                "        if ((threadIdx.x & 63) == 0)",
                "            _base = atomicAdd(&task_counter[0], _tasks_per_wave);",
                "        _base = __shfl(_base, 0, 64);",
                "#endif",
                "        if (_base >= _task_count) return;",
                "        const int _task = _base + (int)(threadIdx.x & 63) / LCD_TASK_LANES;",
                "        bool _pending = _task < _task_count;",
            ]
        records = (protocol == MAILBOX_DEPENDENCE
                   and self._mailbox["gather"] is not None
                   and self._mailbox["gather"].get("records", False))
        incoming = (
            ["        int _mb_next = 0, _mb_end = 0;"] if records else
            ["        int _mb_next = 0, _mb_end = 0;",
             f"        if (_pending) {{ _mb_next = _lcd_in_ptr[{it}]; "
             f"_mb_end = _lcd_in_ptr[{it} + 1]; }}"]
            if protocol == MAILBOX_DEPENDENCE else [])
        if protocol == MAILBOX_DEPENDENCE and self._mailbox["gather"] is not None:
            incoming += self._gather_fetch_lines(2, declare=True,
                                                 records=records)
        node_loads = [
            f"        if (_pending && ({self._prefetch_guard})) {{",
            *[f"            {line}" for line in self._prefetch_lines],
            "        }"]
        chain = self.chain_tasks
        # a chain task walks its members in order; each waits on its own
        # counter, so the position in the chain survives between polls
        member = ([f"{it} = (lcd_index_t)task_nodes[_pos];",
                   f"if ({self._prefetch_guard}) {{",
                   *[f"    {line}" for line in self._prefetch_lines],
                   "}",
                   f"_release_begin = dag_ptr[{it}]; "
                   f"_release_end = dag_ptr[{it} + 1];"] if chain else [])
        lines.append("    const int _tasks_per_wave = 64 / LCD_TASK_LANES;")
        # what a round of tasks starts with is loaded two rounds deep where
        # the later tasks of a wavefront are known in advance: the tiled
        # mailbox with records, the pull protocols on the flat queue
        if (self.pipeline_fetch and tiled and records and self.single_chunk
                and not chain):
            start = self._pipelined_fetch_lines(fetch, it)
        elif (self.pipeline_fetch and not tiled and not chain
              and not self.dynamic_fetch
              and protocol == PULL_DEPENDENCE and self._prefetch_lines
              and (self._value_pull is not None
                   or self._sequential_pull is not None)):
            start = self._pipelined_queue_fetch_lines(it)
        else:
            start = None
        lines += start if start is not None else [
            *fetch,
            *(["        int _pos = 0, _pos_end = 0;",
               "        if (_pending) { _pos = task_ptr[_task]; "
               "_pos_end = task_ptr[_task + 1]; _pending = _pos < _pos_end; }",
               f"        {it} = _pending ? (lcd_index_t)task_nodes[_pos] : 0;"]
              if chain else
              [f"        {it} = 0;"] if records else
              [f"        {it} = _pending ? (lcd_index_t)task_nodes[_task] : 0;"]),
            *(["        if (_pending) { " + " ".join(self._queue_load_lines)
               + " }"] if self._queue_load_lines and not records else []),
            # records are addressed by the queue position: their loads go
            # out with the task id, ahead of the loads that wait for it
            *(incoming + node_loads if records else node_loads),
            *(["        int _release_begin = 0, _release_end = 0;",
               f"        if (_pending) {{ _release_begin = dag_ptr[{it}]; "
               f"_release_end = dag_ptr[{it} + 1]; }}"]
              if protocol == COUNTER_DEPENDENCE else []),
            *([] if records else incoming),
        ]
        value = self._value_pull or self._sequential_pull
        publishes_done = (protocol == PULL_DEPENDENCE
                          and self._value_pull is None
                          and self._published is None)
        if value is not None:
            before, waiting, after = self._value_segments
            # everything ahead of the distributed loop reads nothing another
            # task writes: it runs before the first poll
            lines += ["        if (_pending) {", *task(3, before), "        }"]
        lines += [
            "        unsigned _spins = 0;",
            "        while (__ballot(_pending)) {",
            "            if (_pending) {",
        ]
        if value is not None:
            missing = f"({value['remaining']})"
            none_left = (f"lcd_group_none({missing})"
                         if 1 < self.task_lanes <= 64
                         and self._sequential_pull is None else f"!{missing}")
            lines.append("                bool _ready = true;")
            lines += task(4, waiting + [f"_ready = {none_left};"])
        elif protocol == PULL_DEPENDENCE:
            lines += self._pull_ready_lines(4)
        elif protocol == MAILBOX_DEPENDENCE and self._mailbox["gather"] is not None:
            lines += self._gather_ready_lines(4)
        elif protocol == MAILBOX_DEPENDENCE:
            lines += self._mailbox_ready_lines(4)
        else:
            lines.append(f"                const bool _ready = "
                         f"lcd_load_relaxed(&dep_count[{it}]) == LCD_READY_COUNT;")
        lines.append("                if (_ready) {")
        if value is not None:
            # the last act of the task is the store of its own element:
            # the value is the flag
            lines += task(5, after)
        else:
            lines.append("                    lcd_acquire_fence();")
            lines += task(5)
        if protocol == COUNTER_DEPENDENCE:
            lines += [
                f"                    {self.group_sync}",
                "                    lcd_release_fence();",
                "                    for (int _e = _release_begin + _lane; "
                "_e < _release_end; _e += LCD_TASK_LANES)",
                "                        lcd_atomic_sub(&dep_count[dag_index[_e]], 1);",
            ]
        elif publishes_done:
            lines += [
                f"                    {self.group_sync}",
                "                    lcd_release_fence();",
                f"                    if (_lane == 0) __hip_atomic_store(&done[{it}], 1, "
                "__ATOMIC_RELAXED, LCD_AGENT);",
            ]
        lines += [
            *(["                    if (++_pos < _pos_end) {",
               *[f"                        {line}" for line in member],
               "                    } else {",
               "                        _pending = false;",
               "                    }"] if chain else
              ["                    _pending = false;"]),
            "                } else {",
            "#if LCD_SPIN_SLEEP > 0",
            "                    __builtin_amdgcn_s_sleep(LCD_SPIN_SLEEP);",
            "#endif",
            # the watchdog looks up once in 1024 polls (a 32-bit counter, one
            # test per poll): kept out of the way of the hand-offs, it costs
            # 3 % on the 128^3 grid where the test per poll cost 8 %
            "                    if ((++_spins & 1023u) == 0u && ("
            f"lcd_gave_up(_spins, {STATUS_ARGUMENT}, _lcd_t0) || "
            f"lcd_load_relaxed(&{STATUS_ARGUMENT}[0]) != 0)) {{",
            f"                        {STATUS_ARGUMENT}[0] = 1;",
            "                        _pending = false;",
            "                        _task_aborted = true;",
            "                    }",
            "                }",
            "            }",
            "        }",
            *(["        if (__ballot(_task_aborted)) break;",
               "    }",
               "    if (__syncthreads_or((int)_task_aborted)) return;",
               "    }"] if tiled else
              ["        if (__ballot(_task_aborted)) return;",
               "    }"]),
        ]
        lines.insert(1, "    bool _task_aborted = false;")
        lines.insert(1, "    const long long _lcd_t0 = (long long)wall_clock64();"
                        " (void)_lcd_t0;")
        return lines

    def _reset_kernel_text(self, reset_name):
        """Restores the mutable executor state before every sweep (the
        reference's reset kernel, compiler/cuda_lowering.py:737-853)."""
        values_reset = (
            "    if (t < count) { _lcd_values[2 * t] = LCD_EMPTY_WORD; "
            "_lcd_values[2 * t + 1] = LCD_EMPTY_WORD; }\n"
            "    if (t == 0) { task_counter[0] = 0; }\n",
            "unsigned int* _lcd_values, int* task_counter, long long count")
        if (self.dependence_protocol == MAILBOX_DEPENDENCE
                and self._mailbox["gather"] is not None):
            body, signature = values_reset
        elif self.dependence_protocol == MAILBOX_DEPENDENCE:
            body = ("    if (t < count) { _lcd_mailbox[2 * t] = LCD_EMPTY_WORD; "
                    "_lcd_mailbox[2 * t + 1] = LCD_EMPTY_WORD; }\n"
                    "    if (t == 0) { task_counter[0] = 0; }\n")
            signature = ("unsigned int* _lcd_mailbox, int* task_counter, "
                         "long long count")
        elif (self.dependence_protocol == PULL_DEPENDENCE
              and (self._value_pull is not None or self._published)):
            body = ("    if (t < count) { _lcd_values[2 * t] = LCD_EMPTY_WORD; "
                    "_lcd_values[2 * t + 1] = LCD_EMPTY_WORD; }\n"
                    "    if (t == 0) { task_counter[0] = 0; }\n")
            signature = ("unsigned int* _lcd_values, int* task_counter, "
                         "long long count")
        elif self.dependence_protocol == PULL_DEPENDENCE:
            body = ("    if (t < count) done[t] = 0;\n"
                    "    if (t == 0) { task_counter[0] = 0; }\n")
            signature = ("int* done, int* task_counter, long long count")
        else:
            body = ("    if (t < count) dep_count[t] = initial_dep_count[t];\n"
                    "    if (t == 0) { task_counter[0] = 0; }\n")
            signature = ("int* dep_count, const int* __restrict__ "
                         "initial_dep_count, int* task_counter, long long count")
        return (f'\nextern "C" __global__ void {reset_name}({signature})\n{{\n'
                "    const long long t = (long long)blockIdx.x * blockDim.x + "
                f"threadIdx.x;\n{body}}}\n")

    def _launcher_text(self, launcher_name, kernel_name, reset_name,
                       kernel_arguments):
        """The Python launcher: what the host does on every call."""
        launcher_arguments = []
        for name in kernel_arguments:
            if name in ("band_start", "band_end"):
                if "band_ptr" not in launcher_arguments:
                    launcher_arguments.append("band_ptr")
                continue
            if name in ("task_count", LEVEL_WALKER_LEVELS):
                continue
            launcher_arguments.append(name)
        args = []
        for name in kernel_arguments:
            if name in ("band_start", "band_end"):
                args.append("0")
            elif name == "task_count":
                args.append("_count")
            elif name == LEVEL_WALKER_LEVELS:
                args.append(f"_hip.length({LEVEL_WALKER_ARGUMENTS[0]}) // 64")
            else:
                args.append(name)
        call_args = "(" + ", ".join(args) + ("," if len(args) == 1 else "") + ")"
        body = []
        if self.execution_mode == "plain":
            emitter = self._emitter
            loop = self._target_loop_cache
            body.append(f"_tasks = len(range({', '.join(ast.unparse(a) for a in loop.iter.args)}))")
            body.append(f"_blocks = (_tasks * {self.task_lanes} + "
                        f"{self.threads_per_block} - 1) // {self.threads_per_block}")
            body.append(f"_hip.launch({kernel_name!r}, _blocks, "
                        f"{self.threads_per_block}, {call_args})")
        elif self.execution_mode == "wavefront":
            start = kernel_arguments.index("band_start")
            end = kernel_arguments.index("band_end")
            records = self._level_records
            if records is not None:
                # the right-hand side's share of the node values goes into
                # level order in front of the level launches; the matrix's
                # share and the edge operands only when they have changed
                stage_args = "(" + ", ".join(
                    "_count" if name == "band_end" else text
                    for name, text in zip(kernel_arguments, args)) + ",)"
                static, dynamic = records["kernels"]
                body.append("_count = _hip.length(task_nodes)")
                if records["dynamic"]:
                    body.append(f"_hip.launch({dynamic!r}, (_count + 255) // 256 "
                                f"or 1, 256, {stage_args})")
            body.append(
                f"_hip.launch_levels({kernel_name!r}, band_ptr, "
                f"{max(1, self.threads_per_block // self.task_lanes)}, "
                f"{self.threads_per_block}, {call_args}, {start}, {end})")
            if records is not None:
                restage = [
                    "_count = _hip.length(task_nodes)",
                    f"_hip.launch({static!r}, (_count * {self.record_lanes} + 255) "
                    f"// 256 or 1, 256, {stage_args})"]
                text = (f"def {launcher_name}(_hip, "
                        + ", ".join(launcher_arguments) + "):\n"
                        + "\n".join("    " + line for line in body) + "\n"
                        f"\n\ndef {self._sweep_function_name}_hip_level_restage"
                        "(_hip, " + ", ".join(launcher_arguments) + "):\n"
                        + "\n".join("    " + line for line in restage) + "\n")
                return text, launcher_arguments
        else:
            count_array = {PULL_DEPENDENCE: "done",
                           MAILBOX_DEPENDENCE: "task_nodes"}.get(
                               self.dependence_protocol, "dep_count")
            reset_count = "_count"
            if ((self.dependence_protocol == PULL_DEPENDENCE
                 and (self._value_pull is not None or self._published))
                    or (self.dependence_protocol == MAILBOX_DEPENDENCE
                        and self._mailbox["gather"] is not None)):
                count_array = "task_nodes"
                values = ("_lcd_pub" if self._published else
                          "_lcd_xq" if self._tile is not None
                          and self._tile.get("by_position") else
                          (self._value_pull or self._mailbox)["array"])
                reset_args = (f"({values}, task_counter, "
                              f"_hip.length({values}))")
                reset_count = f"_hip.length({values})"
            elif self.dependence_protocol == PULL_DEPENDENCE:
                reset_args = "(done, task_counter, _hip.length(done))"
            elif self.dependence_protocol == MAILBOX_DEPENDENCE:
                reset_args = ("(_lcd_mailbox, task_counter, "
                              "_hip.length(_lcd_mailbox))")
                reset_count = "_hip.length(_lcd_mailbox)"
            else:
                reset_args = ("(dep_count, initial_dep_count, task_counter, "
                              "_hip.length(dep_count))")
            if self.chain_tasks:
                # tasks are chains; the counters are per node
                reset_count = f"_hip.length({count_array})"
                count_array = "task_ptr"
                body.append("_count = _hip.length(task_ptr) - 1")
            else:
                body.append(f"_count = _hip.length({count_array})")
            if self._walker is None:
                # (a walker polls nothing and writes every element: nothing
                # to restore before a launch)
                body.append(f"_hip.launch({reset_name!r}, ({reset_count} + 255) "
                            f"// 256 or 1, 256, {reset_args})")
            stage_name, stage_arguments = self._stage
            if stage_name is not None:
                for name in stage_arguments:
                    if name not in launcher_arguments:
                        launcher_arguments.append(name)
                stage_args = ", ".join(stage_arguments)
                body.append(
                    f"_hip.launch({stage_name!r}, (_hip.length(_lcd_in_pos) + 255) "
                    f"// 256 or 1, 256, ({stage_args}, _hip.length(_lcd_in_pos)))")
            tasks_per_block = max(1, self.threads_per_block // self.task_lanes)
            waves_per_cu = self.resident_waves_per_cu
            if waves_per_cu is None and not self.block_task:
                # about 64 polling tasks per CU: more slow the producers
                # down, fewer leave hand-off latency exposed (measured on the
                # 128^3 grid with 4 lanes per task and on the power-law
                # matrix with 32)
                waves_per_cu = max(1, self.task_lanes)
                if self._sequential_pull is not None:
                    # tasks that work while they wait (a long body full of
                    # device-coherent loads): about eight per CU measured
                    # best on the 9-point grid (8 lanes per task: 16.2 ms at
                    # one wavefront per CU, 16.8 / 17.6 / 18.4 at 2 / 4 / 8,
                    # 17.5 at one per two CUs; 64 lanes: 10.8 / 10.9 / 11.2
                    # at 6 / 8 / 12)
                    waves_per_cu = max(1, self.task_lanes // 8)
            if self._tile is not None:
                # one workgroup per tile; residency is bounded by the LDS the
                # tile takes, not by a polling budget
                tasks_per_block = self._tile["rows"]
                waves_per_cu = self.resident_waves_per_cu
            if self._sweep is not None:
                # one workgroup per GY x GZ bundles of grid lines; the part of
                # a step's record that is not the matrix's goes in first, the
                # solution comes back out of the wavefronts' order last
                geometry = self._sweep["geometry"]
                blocks = (geometry["slots"] + 255) // 256
                static, dynamic, unstage = self._sweep["kernels"]
                tiles = geometry["tiles"]
                if self._sweep["dynamic_kernel"]:
                    body.append(f"_hip.launch({dynamic!r}, {tiles}, 256, "
                                f"{call_args})")
                body.append(f"_hip.launch({kernel_name!r}, "
                            f"{geometry['workgroups']}, "
                            f"{self.threads_per_block}, {call_args})")
                body.append(f"_hip.launch({unstage!r}, {tiles}, 256, "
                            f"{call_args})")
                restage = [f"_count = _hip.length({count_array})",
                           f"_hip.launch({static!r}, {blocks}, 256, {call_args})"]
                text = (f"def {launcher_name}(_hip, "
                        + ", ".join(launcher_arguments) + "):\n"
                        + "\n".join("    " + line for line in body) + "\n"
                        f"\n\ndef {self._sweep_function_name}_hip_sweep_restage"
                        "(_hip, " + ", ".join(launcher_arguments) + "):\n"
                        + "\n".join("    " + line for line in restage) + "\n")
                return text, launcher_arguments
            if self._walker is not None:
                # one workgroup: the walker and the wavefronts that stage for it
                body.append("_blocks = 1")
            else:
                body.append(f"_blocks = min((_count + {tasks_per_block} - 1) // "
                            f"{tasks_per_block}, _hip.resident_blocks({kernel_name!r}, "
                            f"{self.threads_per_block}, {waves_per_cu!r}))")
            body.append(f"_hip.launch({kernel_name!r}, max(_blocks, 1), "
                        f"{self.threads_per_block}, {call_args})")
        for loop in reversed(self.host_loops):
            header = (f"for {loop.target.id} in "
                      f"{ast.unparse(loop.iter)}:")
            body = [header] + ["    " + line for line in body]
        text = (f"def {launcher_name}(_hip, " + ", ".join(launcher_arguments)
                + "):\n" + "\n".join("    " + line for line in body) + "\n")
        return text, launcher_arguments


def lower_to_hip(code, loop_iterator, reductions=None, kernel_name=None,
                 execution_mode="plain", sync_free_ready_count=0,
                 wavefront_threads_per_block=128, thread_loop_iterator=None,
                 thread_unroll_factor=1, n_warp=None,
                 dependence_protocol=COUNTER_DEPENDENCE, direct_dependence=None,
                 function_props=None, structural_lookups=(), task_lanes=None,
                 chain_tasks=False, argument_kinds=None,
                 spin_limit=DEFAULT_SPIN_LIMIT, resident_waves_per_cu=None,
                 spin_sleep=1, promote_own_elements=True,
                 prefetch_node_loads=True, value_flags=True,
                 gather_messages=True, segment_cache=True, tile_rows=None,
                 stage_operands=True, task_records=True, single_chunk=False,
                 queue_node_loads=True, plain_first_polls=None,
                 publish_values=True, look_ahead=True, segment_capacity=None,
                 pipeline_fetch=True, full_fences=False, dynamic_fetch=False,
                 tile_positions=None, tile_by_position=False,
                 segment_registers=False, pair_tables=True, band_walker=False,
                 level_walker=0, prepared_division=True, grid_sweep=None,
                 watchdog_seconds=None, level_records=True):
    """HIP counterpart of ``lower_to_numba_cuda``
    (compiler/cuda_lowering.py:2854-2884); same parameters plus
    ``task_lanes`` (lanes cooperating on one task, a power of two <= 64),
    ``chain_tasks`` (tasks are node sequences, ``band_width > 1``) and
    ``spin_limit`` (watchdog of the sync-free poll loop)."""
    lowerer = HIPLowerer(
        loop_iterator=loop_iterator, reductions=reductions,
        kernel_name=kernel_name, execution_mode=execution_mode,
        sync_free_ready_count=sync_free_ready_count,
        wavefront_threads_per_block=wavefront_threads_per_block,
        thread_loop_iterator=thread_loop_iterator,
        thread_unroll_factor=thread_unroll_factor, n_warp=n_warp,
        dependence_protocol=dependence_protocol,
        direct_dependence=direct_dependence, function_props=function_props,
        structural_lookups=structural_lookups, task_lanes=task_lanes,
        chain_tasks=chain_tasks, argument_kinds=argument_kinds,
        spin_limit=spin_limit, resident_waves_per_cu=resident_waves_per_cu,
        spin_sleep=spin_sleep, promote_own_elements=promote_own_elements,
        prefetch_node_loads=prefetch_node_loads, value_flags=value_flags,
        gather_messages=gather_messages, segment_cache=segment_cache,
        tile_rows=tile_rows, stage_operands=stage_operands,
        task_records=task_records, single_chunk=single_chunk,
        queue_node_loads=queue_node_loads,
        plain_first_polls=plain_first_polls, publish_values=publish_values,
        look_ahead=look_ahead, segment_capacity=segment_capacity,
        pipeline_fetch=pipeline_fetch, full_fences=full_fences,
        dynamic_fetch=dynamic_fetch, tile_positions=tile_positions,
        tile_by_position=tile_by_position,
        segment_registers=segment_registers, pair_tables=pair_tables,
        band_walker=band_walker, level_walker=level_walker,
        prepared_division=prepared_division, grid_sweep=grid_sweep,
        watchdog_seconds=watchdog_seconds, level_records=level_records)
    return lowerer.lower(code)

"""Schedule space, workload features and the analytic scheduler for MI355X.

Counterpart of compiler/scheduler.py of the reference (space :172-303, cost
model :306-419, features :422-452, trip-count probe :455-571, fingerprint
:678-711, machine constants :714-775), re-fitted to CDNA4:

* a wavefront is 64 lanes (``WAVE_SIZE``); ``n_warp`` counts cooperating
  wavefronts;
* a thread-mapped task may use a *slice* of a wavefront: ``task_lanes`` is an
  extra schedule dimension (4..64 lanes), searched when the user fixes neither
  ``n_warp`` nor ``task_lanes``;
* the level loop of the wavefront executor is replayed from a hipGraph, so its
  per-level cost is the measured graph-node cost, not a host launch;
* the sync-free estimate includes the dependency critical path
  ``levels * handoff``, the measured cross-workgroup release/acquire latency;
* machine constants are measured by ``lcdhip_measure_arch`` on the device.
"""

import ast
import hashlib
import itertools
import math
from copy import deepcopy
from dataclasses import dataclass, replace

import numpy as np

try:
    import xxhash as _xxhash
except ImportError:        # pragma: no cover - depends on the image
    _xxhash = None

from lcd_amd.dag_codegen import (
    COUNTER_DEPENDENCE,
    MAILBOX_DEPENDENCE,
    PULL_DEPENDENCE,
    PUSH_DEPENDENCE,
)

WAVEFRONT = "wavefront"
SYNC_FREE = "sync_free"
AUTO = "auto"
EXECUTION_MODES = (WAVEFRONT, SYNC_FREE)
BLOCK_SIZES = (64, 128, 256, 512)
UNROLL_FACTORS = (1, 2, 4, 8)
DEFAULT_THREADS_PER_BLOCK = 128
N_WARP_CANDIDATES = (1,)
WAVE_SIZE = 64
TASK_LANE_CANDIDATES = (4, 8, 16, 32, 64)
PULL_POLLING_FACTOR = 2.0
ARITHMETIC_OPERATORS = (ast.Add, ast.Sub, ast.Mult, ast.Div, ast.FloorDiv,
                        ast.Mod, ast.Pow)


class SchedulerError(Exception):
    pass


@dataclass(frozen=True)
class ArchConstants:
    launch_latency_s: float
    atomic_cost_s: float
    memory_bandwidth_bytes_per_s: float
    lane_flops_per_s: float
    handoff_s: float = 0.0        # release -> acquire between workgroups
    barrier_s: float = 0.0        # one grid barrier of a resident grid
    graph_node_s: float = 0.0     # one dependent kernel node of a hipGraph
    lds_handoff_s: float = 0.0    # the hop between wavefronts of one workgroup
    chain_step_s: float = 0.0     # one dependent fp64 task, hand-off free


# The mailbox protocol's level time on a busy MI355X: 3.3 x the idle-GPU
# hand-off (0.54 us -> 1.8 us per level from 1800 rows per level on), and
# about 5.3 G tasks/s once levels are wider than that (192^3 grid: 2.4 us
# per level of 12 K rows; 256^3: 3.8 us per level of 22 K rows).
LOADED_HANDOFF_FACTOR = 3.3
TASK_ISSUE_S = 1.9e-10

# Used when no device is available to measure (MI355X data-sheet scale).
FALLBACK_ARCH_CONSTANTS = ArchConstants(
    launch_latency_s=8.0e-6,
    atomic_cost_s=2.0e-9,
    memory_bandwidth_bytes_per_s=8.0e12,
    lane_flops_per_s=2.4e9,
    handoff_s=1.5e-6,
    barrier_s=4.0e-6,
    graph_node_s=2.5e-6,
)


@dataclass(frozen=True)
class WorkloadFeatures:
    rows: int
    edges: int
    levels: int
    nonzeros: int
    flops: float
    memory_bytes: int
    thread_work_items: int = 0
    thread_loop_invocations: int = 0
    # sum of squared trip counts of the mapped loop (0 = not known): with it
    # the trip count seen from a work item, sum t^2 / sum t, tells skewed
    # segment lengths from uniform ones
    thread_work_squares: int = 0

    @property
    def average_in_degree(self):
        return 0.0 if self.rows == 0 else self.edges / self.rows

    @property
    def average_thread_trip_count(self):
        if self.thread_loop_invocations == 0:
            return 0.0
        return self.thread_work_items / self.thread_loop_invocations

    @property
    def weighted_thread_trip_count(self):
        """Trip count of the segment an average work item belongs to."""
        if self.thread_work_items == 0 or self.thread_work_squares == 0:
            return self.average_thread_trip_count
        return self.thread_work_squares / self.thread_work_items


@dataclass(frozen=True)
class CostEstimate:
    launch_s: float
    sync_s: float
    memory_s: float
    compute_s: float

    @property
    def total_s(self):
        return self.launch_s + self.sync_s + self.memory_s + self.compute_s


@dataclass(frozen=True)
class Schedule:
    execution_mode: str
    threads_per_block: int
    thread_unroll: int
    n_warp: int = 1
    dependence_protocol: str = COUNTER_DEPENDENCE
    task_lanes: int = 0           # 0: the default group (a whole wavefront)
    cost: CostEstimate | None = None

    @property
    def lowering_key(self):
        return (self.execution_mode, self.threads_per_block,
                self.thread_unroll, self.n_warp, self.dependence_protocol,
                self.task_lanes)


@dataclass(frozen=True)
class SchedulePlan:
    schedule: Schedule
    execution_data: object
    features: WorkloadFeatures | None = None
    dag: object = None
    tile_rows: int | None = None     # tiled persistent executor, or None
    single_chunk: bool = False       # no task has more in-edges than lanes
    task_records: bool = True        # record arrays fit 32-bit indices
    tile_boxes: tuple | None = None  # (grid, box): tiles are boxes of a grid
    # own segments (<= 64 entries) in registers: 0 no, 1 yes, 2 with the
    # structure searches of the producer loop read from tables
    segment_registers: int = 0
    # one wavefront runs the tasks in program order (chain-like DAGs)
    band_walker: bool = False
    # one wavefront takes a level per step (small DAGs with narrow levels):
    # the incoming entries per task it has room for, or 0
    level_walker: int = 0
    # the grid sweep: (nx, ny, nz, WY, GY, GZ, SKZ), or None
    grid_sweep: tuple | None = None
    # what the scheduler has to say about the plan beyond the schedule (a
    # DAG that belongs on the host), or None
    advice: str | None = None


# Grid sweep, automatic choice (WY, GY, GZ, SKZ): bundles of 8 x 8 grid lines
# per wavefront, two bundles stacked along z per workgroup, one step between
# the z rows of a bundle.  Measured on the 128^3 grid (one solve: staging of
# the right-hand side, sweep, solution back to its array): 125 us with this
# shape; 126 us with the two bundles side by side along y; 128 us with one
# bundle per workgroup (more faces through memory); 139 us with four (four
# streams of operands share one CU's path to memory); 132 us with bundles of
# 16 x 4 lines; two steps between the z rows (the z value is then read from
# LDS a step ahead of its use, but a bundle takes 14 steps more and the path
# through the grid 127) 143 us with 8 x 8 lines and 162 us with 16 x 4.
GRID_SWEEP_SHAPE = (8, 1, 2, 1)


# Tiled executor, automatic choice: tiles of 4096 consecutive block-iterator
# values (32 KB of LDS, two workgroups of six wavefronts per CU; 384 threads
# measured best on the 128^3 grid: 0.485 ms against 0.53 at 256 and 0.49 at
# 512) once the problem has at least
# four of them, a quarter of the problem below that; only when at least half
# of the DAG's edges stay inside a tile (measured: the 128^3 grid keeps 2/3
# and runs 1.25-1.45 x faster tiled, a random power-law matrix keeps none and
# runs 10 x slower).
TILE_ROWS = 4096
TILE_MIN_ROWS = 256
TILE_MIN_LOCALITY = 0.5
TILE_THREADS_PER_BLOCK = 384
# Box tiles keep their eight wavefronts busy (whole lines: 32 tasks per level,
# two wavefronts per level, four levels in flight): 128^3 with boxes of
# 128 x 8 x 4 runs in 0.287 / 0.247 / 0.238 / 0.305 ms at 256 / 384 / 512 / 640
# threads.
TILE_BOX_THREADS_PER_BLOCK = 512
# Once there are more such tiles than workgroups of 384 threads can be
# resident (three per CU on 256 CUs), the solve is bound by throughput rather
# than by hand-offs, and more, smaller tiles with fewer threads each measured
# faster: 256^3 grid 1.91 ms with 2048 rows and 128 threads against 2.37 ms,
# 192^3 1.05 against 1.23 ms; the 128^3 grid the other way round, 0.52 against
# 0.33 ms.  Only with wide levels, though: a 2048^2 grid has as many rows as
# the 160^3 one but 4095 levels of at most 2048 rows, stays bound by
# hand-offs and keeps the large tiles (3.86 ms against 4.07 ms).
TILE_LARGE_PROBLEM_ROWS = 768 * TILE_ROWS
TILE_LARGE_PROBLEM_WIDTH = 8192
TILE_LARGE_ROWS = 2048
TILE_LARGE_THREADS_PER_BLOCK = 128


def _throughput_bound(dag):
    levels = max(int(getattr(dag, "levels", 0) or 0), 1)
    return (dag.n > TILE_LARGE_PROBLEM_ROWS
            and dag.n / levels >= TILE_LARGE_PROBLEM_WIDTH)


def automatic_tile_threads(dag):
    """Threads per tile that go with ``automatic_tile_rows``."""
    return (TILE_LARGE_THREADS_PER_BLOCK if _throughput_bound(dag)
            else TILE_THREADS_PER_BLOCK)


def automatic_tile_rows(dag):
    """Tile size for this DAG, or None when tiles would not pay."""
    if not getattr(dag, "topological_ids", False) or dag.n < 4 * TILE_MIN_ROWS:
        return None
    rows = TILE_LARGE_ROWS if _throughput_bound(dag) else TILE_ROWS
    while rows > TILE_MIN_ROWS and dag.n < 4 * rows:
        rows //= 2
    if dag.tile_locality(rows) < TILE_MIN_LOCALITY:
        return None
    return rows


# Pair tables hold one entry per pair of positions of a segment (9-point grid:
# 81 per row, 8.6 per stored position; 64 at most with segments of up to 64
# entries).  Beyond this many per stored position the structure keeps its
# searches in the kernel.
PAIR_TABLE_ENTRIES_PER_POSITION = 24


# Tiles of the published pull (ILU0), automatic choice: a tile's slice of the
# publication buffer has a copy of 9216 entries in LDS (72 KB: two workgroups
# per CU), so a tile holds 0.9 x 9216 / (mean row length) rows; ten wavefronts
# per tile; only where at least a fifth of the DAG's edges stay inside such a
# tile (the 9-point grid keeps one in four: the row before).
PUBLISHED_TILE_POSITIONS = 9216
PUBLISHED_TILE_THREADS_PER_BLOCK = 640
PUBLISHED_TILE_MIN_LOCALITY = 0.2

# Band walker, automatic choice.  One wavefront runs the tasks in program
# order at about 0.06 us per task whatever the DAG looks like; the persistent
# executors pay one hand-off (0.4 us in a tile) per LEVEL.  The walker wins
# once a level holds fewer than about seven tasks; it is chosen at fewer than
# six.  Its table of coefficients has a cell per (source, lane): every edge
# must span fewer than 64 iterations.  (The 4 M-row band of width 8: 0.25 s
# against 1.79 s in tiles of 8192 rows.)
BAND_WALKER_TASKS_PER_LEVEL = 6
BAND_WALKER_SPAN = 64
BAND_WALKER_THREADS_PER_BLOCK = 1024


class SchedulerAdvice(UserWarning):
    """The plan will run, but the scheduler expects another place to be
    faster (see ``SchedulePlan.advice``)."""


# A DAG that is close to a chain has nothing to run in parallel: the GPU pays
# its per-task cost in sequence -- 0.06 us on the band walker (143 cycles: the
# dependent arithmetic of a row and what one wavefront issues beside it),
# 0.43 us per level in tiles when an edge is too long for the walker -- where
# one host core runs the compiled loop at about 1.2 ns per stored entry (the
# single-threaded C restatement: 30 ms for the 4 M-row band of width 8,
# against 250 ms on the walker).  The estimates only have to tell 8 x apart.
BAND_WALKER_SECONDS_PER_TASK = 6.0e-8
TILED_SECONDS_PER_LEVEL = 4.3e-7
HOST_LOOP_SECONDS_PER_ENTRY = 1.2e-9
HOST_LOOP_SECONDS_PER_TASK = 2.0e-9
SEQUENTIAL_ADVICE_MIN_TASKS = 10000


def sequential_advice(dag, band_walker=False):
    """Text for ``SchedulePlan.advice`` when the DAG is so close to a chain
    (fewer than BAND_WALKER_TASKS_PER_LEVEL tasks per level) that a compiled
    sequential loop on one host core is expected to beat the GPU, else None.
    The plan still runs on the GPU: the caller may have its data there."""
    levels = int(getattr(dag, "levels", 0) or 0)
    if (dag.n < SEQUENTIAL_ADVICE_MIN_TASKS
            or levels * BAND_WALKER_TASKS_PER_LEVEL <= dag.n):
        return None
    device = (dag.n * BAND_WALKER_SECONDS_PER_TASK if band_walker
              else levels * TILED_SECONDS_PER_LEVEL)
    host = (dag.n * HOST_LOOP_SECONDS_PER_TASK
            + (dag.edges + dag.n) * HOST_LOOP_SECONDS_PER_ENTRY)
    if device <= 2.0 * host:
        return None
    return (
        f"the dependence DAG is close to a chain ({levels} levels for "
        f"{dag.n} iterations): nothing runs in parallel, and the GPU is "
        f"expected to take about {device * 1e3:.3g} ms per call "
        f"({'one wavefront in program order' if band_walker else 'one hand-off per level'}"
        f") where a compiled sequential loop on one host core takes about "
        f"{host * 1e3:.3g} ms; the call runs on the GPU all the same")


def band_walker_applies(dag, forced=False):
    """True when the DAG is close enough to a chain for the band walker
    (always, when ``forced``) and every edge spans fewer than 64 iterations
    (destination - source in 1 .. 63)."""
    if dag.n == 0 or dag.edges == 0:
        return False
    if not forced and dag.levels * BAND_WALKER_TASKS_PER_LEVEL <= dag.n:
        return False
    offsets, _, distinct = dag.edge_offsets(BAND_WALKER_SPAN)
    return (0 < distinct < BAND_WALKER_SPAN and offsets[0] >= 1
            and offsets[-1] < BAND_WALKER_SPAN)


# Level walker, automatic choice: a DAG small enough for its values to live in
# one workgroup's LDS (4096 tasks) whose tasks have at most four incoming
# entries.  One wavefront then takes a step of up to 64 tasks of one level in
# about 0.15 us (369 cycles measured on the 64 x 64 grid of configuration 1,
# 127 levels) where the persistent executors pay a polled hand-off of 0.5 us
# per level; a level of more than 64 tasks takes several steps, and the
# walker is chosen while it has at most three steps per level on average.
LEVEL_WALKER_WIDTH = 64
LEVEL_WALKER_STEPS_PER_LEVEL = 3


def level_walker_records(dag, max_tasks, max_entries, forced=False):
    """The structure step-major for the level walker -- ``(entries, task,
    source, position)`` with ``task[step * 64 + lane]``, ``source`` and
    ``position[(step * entries + k) * 64 + lane]`` (-1: no task, no entry;
    the dummy source is ``max_tasks``); a step is up to 64 tasks of one level
    (tasks of a level do not depend on each other) -- or None when the DAG
    does not fit: more than ``max_tasks`` tasks, a task with more than
    ``max_entries`` incoming entries, or (unless ``forced``) more than
    LEVEL_WALKER_STEPS_PER_LEVEL steps per level on average.  Built on the
    host: the DAG is small by definition."""
    if dag.n == 0 or dag.n > max_tasks or dag.edges == 0:
        return None
    pointer = np.asarray(dag.host("wavefront_ptr"), dtype=np.int64)
    widths = np.diff(pointer)
    if len(widths) == 0:
        return None
    chunks = -(-widths // LEVEL_WALKER_WIDTH)
    steps = int(chunks.sum())
    if not forced and steps > LEVEL_WALKER_STEPS_PER_LEVEL * len(widths):
        return None
    in_ptr = np.asarray(dag.host("in_ptr"), dtype=np.int64)
    counts = np.diff(in_ptr)
    entries = int(counts.max()) if len(counts) else 0
    if entries < 1 or entries > max_entries:
        return None
    nodes = np.asarray(dag.host("wavefronts"), dtype=np.int64)
    in_src = np.asarray(dag.host("in_src"), dtype=np.int32)
    in_pos = np.asarray(dag.host("in_pos"), dtype=np.int32)
    level_of = np.repeat(np.arange(len(widths)), widths)
    within = np.arange(len(nodes)) - pointer[level_of]
    first_step = np.concatenate([[0], np.cumsum(chunks)[:-1]])
    step_of = first_step[level_of] + within // LEVEL_WALKER_WIDTH
    lane_of = within % LEVEL_WALKER_WIDTH
    task = np.full(steps * 64, -1, dtype=np.int32)
    task[step_of * 64 + lane_of] = nodes
    source = np.full(steps * entries * 64, max_tasks, dtype=np.int32)
    position = np.full(steps * entries * 64, -1, dtype=np.int32)
    for k in range(entries):
        has = counts[nodes] > k
        at = (step_of[has] * entries + k) * 64 + lane_of[has]
        which = in_ptr[nodes[has]] + k
        source[at] = in_src[which]
        position[at] = in_pos[which]
    return entries, task, source, position


def structured_grid(dag):
    """``(nx, ny, nz)`` when the DAG's edges are those of an axis stencil on
    a grid in natural order (id = x + nx * (y + ny * z)): every edge goes
    from a node to its neighbour one step up along an axis, so destination -
    source takes the values 1, nx and nx * ny (1 and nx in two dimensions)
    and nothing else.  None for every other structure.  The answer picks a
    task order, never a result: an order that is not topological is refused
    when the task records are built."""
    offsets, counts, distinct = dag.edge_offsets(4)
    if distinct not in (2, 3) or offsets[0] != 1:
        return None
    line = offsets[1]
    plane = offsets[2] if distinct == 3 else dag.n
    if line < 2 or plane % line or plane // line < 2 or dag.n % plane:
        return None
    grid = (line, plane // line, dag.n // plane)
    # a full stencil has one edge per node and axis, less the upper faces
    expected = [dag.n // grid[axis] * (grid[axis] - 1) for axis in range(3)]
    if list(counts) != expected[:distinct]:
        return None
    return grid


def automatic_tile_box(grid, rows):
    """Box extents for tiles of at most ``rows`` points over a structured
    grid, or None when boxes would be tiles of consecutive ids anyway.

    A box takes whole lines along x and splits what is left between y and z
    (powers of two) so that the critical path crosses the fewest box faces,
    sum(grid / box - 1) of them, each a hand-off through memory instead of
    LDS.  Whole lines keep the level sets of a box narrow (by * bz tasks) and
    many (nx + by + bz - 2), which is what the wavefronts of a tile want:
    measured on the 128^3 grid with 4096 points per box, 128 x 8 x 4 runs in
    0.247 ms, 64 x 8 x 8 in 0.348, 32 x 8 x 16 in 0.590 and 16 x 16 x 16 --
    the fewest crossings of all -- in 0.792, against 0.318 ms for 32
    consecutive lines of one plane."""
    nx, ny, nz = grid
    lines = rows // nx
    if lines < 2 or nz < 2:
        return None

    def extents(limit):
        values, extent = [], 1
        while extent < limit:
            values.append(extent)
            extent *= 2
        return values + [limit]

    best, best_key = None, None
    for by in extents(ny):
        for bz in extents(nz):
            if by * bz > lines:
                continue
            crossings = -(-ny // by) + -(-nz // bz) - 2
            key = (crossings, -by * bz, -by)
            if best_key is None or key < best_key:
                best, best_key = (nx, by, bz), key
    return best if best[2] > 1 else None


def normalize_execution_mode(execution_mode):
    if execution_mode is None or execution_mode == AUTO:
        return None
    if execution_mode.replace("-", "_") == SYNC_FREE:
        return SYNC_FREE
    return WAVEFRONT


def task_threads(threads_per_block, n_warp, task_lanes=0):
    """Lanes that cooperate on one task."""
    if task_lanes:
        return task_lanes
    if threads_per_block % WAVE_SIZE:
        return threads_per_block
    return min(threads_per_block, WAVE_SIZE * n_warp)


def _wave_task(threads_per_block, n_warp):
    return n_warp == 1 and threads_per_block % WAVE_SIZE == 0


@dataclass(frozen=True)
class ScheduleSpace:
    execution_modes: tuple
    block_sizes: tuple
    unroll_factors: tuple
    n_warps: tuple = N_WARP_CANDIDATES
    thread_mapped: bool = False
    dependence_protocols: tuple = (COUNTER_DEPENDENCE,)
    task_lanes: tuple = (0,)
    # the pull protocol waits inside a sequential loop of the task: tasks
    # that share a wavefront then serialise each other's work between polls,
    # so such a task gets a wavefront of its own (ILU0, 9-point grid:
    # 14.1 ms with 8 lanes per task, 10.9 ms with 64)
    sequential_pull: bool = False
    # level launches of a push-shaped loop gather their incoming products
    # instead of pushing them with atomics (the mailbox protocol's listing,
    # without polls): deterministic sums, bit-identical to the sequential loop
    level_gather: bool = False

    @classmethod
    def from_options(cls, execution_mode=None, threads_per_block=None,
                     thread_unroll=None, thread_mapped=False, n_warp=None,
                     direct_protocol=None, dependence_protocol=None,
                     task_lanes=None, sequential_pull=False,
                     level_gather=False):
        mode = normalize_execution_mode(execution_mode)
        if n_warp is not None and (not isinstance(n_warp, int) or n_warp <= 0):
            raise SchedulerError("n_warp must be a positive integer.")
        block_task = n_warp is not None and n_warp > 1
        if (block_task and threads_per_block is not None
                and threads_per_block != n_warp * WAVE_SIZE):
            raise SchedulerError(
                f"n_warp={n_warp} maps one task to {n_warp * WAVE_SIZE} "
                f"threads, but threads_per_block={threads_per_block}.")
        if (n_warp == 1 and thread_mapped and threads_per_block is not None
                and threads_per_block % WAVE_SIZE):
            raise SchedulerError(
                "n_warp=1 requires threads_per_block to be a multiple of "
                f"{WAVE_SIZE}, but threads_per_block={threads_per_block}.")
        if task_lanes is not None:
            if (not isinstance(task_lanes, int) or task_lanes <= 0
                    or task_lanes & (task_lanes - 1) or task_lanes > WAVE_SIZE):
                raise SchedulerError(
                    "task_lanes must be a power of two between 1 and "
                    f"{WAVE_SIZE}.")
            if block_task:
                raise SchedulerError(
                    "task_lanes cannot be combined with n_warp > 1.")
        if threads_per_block is not None:
            block_sizes = (threads_per_block,)
        elif block_task:
            block_sizes = (n_warp * WAVE_SIZE,)
        elif thread_mapped:
            block_sizes = BLOCK_SIZES
        else:
            block_sizes = (DEFAULT_THREADS_PER_BLOCK,)
        if thread_unroll is not None:
            unroll_factors = (thread_unroll,)
        elif thread_mapped:
            unroll_factors = UNROLL_FACTORS
        else:
            unroll_factors = (1,)
        if not thread_mapped or block_task:
            lanes = (0,)
        elif task_lanes is not None:
            lanes = (task_lanes,)
        elif n_warp == 1:
            lanes = (0,)                 # one whole wavefront per task
        else:
            lanes = TASK_LANE_CANDIDATES
        execution_modes = EXECUTION_MODES if mode is None else (mode,)
        n_warps = N_WARP_CANDIDATES if n_warp is None else (n_warp,)
        available = (COUNTER_DEPENDENCE,) + (
            (direct_protocol,)
            if thread_mapped and direct_protocol is not None else ())
        if PUSH_DEPENDENCE in available:
            available += (MAILBOX_DEPENDENCE,)
        searched = (len(execution_modes) * len(block_sizes)
                    * len(unroll_factors) * len(n_warps) * len(lanes)) > 1
        if dependence_protocol is not None:
            if dependence_protocol not in available:
                raise SchedulerError(
                    f"Dependence protocol {dependence_protocol!r} is not "
                    "supported by this loop; available protocols: "
                    + ", ".join(available) + ".")
            protocols = (dependence_protocol,)
        elif PUSH_DEPENDENCE in available:
            # message slots beat atomics + counters wherever a push applies
            # (one hop per edge, deterministic sums); the lowering falls back
            # to the push protocol for loop shapes the mailbox cannot express
            protocols = (MAILBOX_DEPENDENCE,)
        elif PULL_DEPENDENCE in available and sequential_pull:
            # waiting for each producer where it is used beats waiting for
            # all of them up front (ILU0: 10.9 ms against 35 ms); the
            # lowering falls back to counters for loops it cannot resume
            protocols = (PULL_DEPENDENCE,)
        elif PULL_DEPENDENCE in available and searched:
            protocols = (COUNTER_DEPENDENCE, PULL_DEPENDENCE)
        else:
            protocols = (COUNTER_DEPENDENCE,)
        return cls(execution_modes=execution_modes, block_sizes=block_sizes,
                   unroll_factors=unroll_factors, n_warps=n_warps,
                   thread_mapped=thread_mapped,
                   dependence_protocols=protocols, task_lanes=lanes,
                   sequential_pull=bool(sequential_pull),
                   level_gather=bool(level_gather)
                   and MAILBOX_DEPENDENCE in protocols)

    def configurations(self):
        result = []
        for mode, block, unroll, n_warp, lanes in itertools.product(
                self.execution_modes, self.block_sizes, self.unroll_factors,
                self.n_warps, self.task_lanes):
            if lanes and block % lanes:
                continue
            protocols = (
                self.dependence_protocols
                if (mode == SYNC_FREE and self.thread_mapped
                    and _wave_task(block, n_warp))
                else (MAILBOX_DEPENDENCE,)
                if (self.level_gather and self.thread_mapped
                    and _wave_task(block, n_warp))
                # level launches of a sequential producer loop, a wavefront
                # per task: the pull executor's task with plain loads (the
                # lowering keeps the counters where it does not apply)
                else (PULL_DEPENDENCE,)
                if (mode == WAVEFRONT and self.sequential_pull
                    and self.thread_mapped
                    and PULL_DEPENDENCE in self.dependence_protocols
                    and lanes in (0, WAVE_SIZE) and block >= WAVE_SIZE
                    and _wave_task(block, n_warp))
                else (COUNTER_DEPENDENCE,))
            for protocol in protocols:
                if (protocol == PULL_DEPENDENCE and self.sequential_pull
                        and lanes not in (0, WAVE_SIZE)
                        and WAVE_SIZE in self.task_lanes):
                    continue
                result.append((mode, block, unroll, n_warp, protocol, lanes))
        return result

    @property
    def is_fixed(self):
        return len(self.configurations()) == 1

    def fixed_schedule(self):
        if not self.is_fixed:
            raise SchedulerError(
                "The schedule space has more than one configuration.")
        return Schedule(*self.configurations()[0])


class AnalyticScheduler:
    def __init__(self, arch_constants=None):
        self._arch_constants = arch_constants

    @property
    def arch_constants(self):
        if self._arch_constants is None:
            self._arch_constants = measure_arch_constants()
        return self._arch_constants

    def estimate(self, features, execution_mode, threads_per_block,
                 thread_unroll, n_warp, thread_mapped,
                 dependence_protocol=COUNTER_DEPENDENCE, task_lanes=0):
        arch = self.arch_constants
        average_in_degree = features.average_in_degree
        if execution_mode == WAVEFRONT:
            per_level = arch.graph_node_s or arch.launch_latency_s
            launch_s = features.levels * per_level
            sync_s = 0.0
        elif execution_mode == SYNC_FREE:
            launch_s = arch.launch_latency_s
            if dependence_protocol == MAILBOX_DEPENDENCE:
                # no atomics: a level costs one hand-off under load, or the
                # issue time of its tasks when it is wide
                width = features.rows / max(features.levels, 1)
                sync_s = features.levels * max(
                    (LOADED_HANDOFF_FACTOR - 1.0) * arch.handoff_s,
                    width * TASK_ISSUE_S - arch.handoff_s)
            elif dependence_protocol == PUSH_DEPENDENCE:
                sync_s = arch.atomic_cost_s * features.rows / n_warp
            elif dependence_protocol == PULL_DEPENDENCE:
                sync_s = arch.atomic_cost_s * average_in_degree * (
                    1.0 + PULL_POLLING_FACTOR * features.levels)
            else:
                sync_s = arch.atomic_cost_s * (
                    average_in_degree + features.rows / n_warp)
            sync_s += features.levels * arch.handoff_s
        else:
            raise SchedulerError(f"Unknown execution mode {execution_mode!r}.")
        lanes = (task_threads(threads_per_block, n_warp, task_lanes)
                 * thread_unroll if thread_mapped else 1)
        parallelism = (self.lane_parallelism(features)
                       if thread_mapped and features.thread_loop_invocations
                       else average_in_degree)
        active_lanes = min(lanes, max(parallelism, 1.0))
        return CostEstimate(
            launch_s=launch_s, sync_s=sync_s,
            memory_s=features.memory_bytes / arch.memory_bandwidth_bytes_per_s,
            compute_s=features.flops / (active_lanes * arch.lane_flops_per_s))

    def lane_parallelism(self, features):
        """Lanes a task of the mapped loop can keep busy."""
        return features.average_thread_trip_count

    def candidates(self, features, space):
        return [
            Schedule(mode, block, unroll, n_warp, protocol, lanes,
                     cost=self.estimate(features, mode, block, unroll, n_warp,
                                        space.thread_mapped, protocol, lanes))
            for mode, block, unroll, n_warp, protocol, lanes
            in space.configurations()]

    def schedule(self, features, space):
        return min(self.candidates(features, space), key=_schedule_rank)


class CalibratedScheduler(AnalyticScheduler):
    """The analytic model with its latency terms scaled to what the
    executors measure on MI355X (the decorator's default).

    The reference's formulas price a level of the level-synchronous executor
    at one launch and a hand-off of the persistent executor at one idle
    release -> acquire.  Measured here: a level kernel's dependent loads make
    a level 2.3 x the bare graph node (3.9 us on the 128^3 grid); a busy GPU
    stretches the hand-off 3.3 x, and the protocols differ in how many
    device-scope hops one level takes (message slots and value-flagged pulls
    one, atomics + counters or flags about 1.6 x that, plain counters more,
    since the task body then reads its operands through coherent loads)."""

    LEVEL_KERNEL_FACTOR = 2.3
    # a wide level is bound by its rows, not by the launch: 3.9 us per level
    # at 5.5 K rows per level (128^3 grid), 7.5 us at 22 K (256^3), i.e.
    # 1.6 graph nodes + 0.215 ns per row
    WIDE_LEVEL_FACTOR = 1.6
    LEVEL_ROW_S = 2.15e-10
    HANDOFFS_PER_LEVEL = {
        MAILBOX_DEPENDENCE: LOADED_HANDOFF_FACTOR,
        PULL_DEPENDENCE: LOADED_HANDOFF_FACTOR,
        PUSH_DEPENDENCE: 1.6 * LOADED_HANDOFF_FACTOR,
        COUNTER_DEPENDENCE: 2.4 * LOADED_HANDOFF_FACTOR,
    }

    def lane_parallelism(self, features):
        """Geometric mean of the plain and the work-weighted trip count: with
        uniform segments both agree; with power-law rows (n = 10^6, mean 17,
        work-weighted 134) the long rows carry the critical path, and 32 to 64
        lanes measured 20 % faster than the 16 the plain mean selects."""
        return math.sqrt(features.average_thread_trip_count
                         * features.weighted_thread_trip_count)

    def estimate(self, features, execution_mode, threads_per_block,
                 thread_unroll, n_warp, thread_mapped,
                 dependence_protocol=COUNTER_DEPENDENCE, task_lanes=0):
        base = super().estimate(features, execution_mode, threads_per_block,
                                thread_unroll, n_warp, thread_mapped,
                                dependence_protocol, task_lanes)
        arch = self.arch_constants
        if execution_mode == WAVEFRONT:
            wide_s = (base.launch_s * self.WIDE_LEVEL_FACTOR
                      + features.rows * self.LEVEL_ROW_S)
            return replace(base, launch_s=max(
                base.launch_s * self.LEVEL_KERNEL_FACTOR, wide_s))
        hops = self.HANDOFFS_PER_LEVEL.get(dependence_protocol,
                                           LOADED_HANDOFF_FACTOR)
        if dependence_protocol == MAILBOX_DEPENDENCE:
            return base      # already priced under load
        return replace(base, sync_s=base.sync_s
                       + (hops - 1.0) * features.levels * arch.handoff_s)


def _schedule_rank(schedule):
    return (
        schedule.cost.total_s,
        task_threads(schedule.threads_per_block, schedule.n_warp,
                     schedule.task_lanes) * schedule.thread_unroll,
        abs(schedule.threads_per_block.bit_length()
            - DEFAULT_THREADS_PER_BLOCK.bit_length()),
        schedule.threads_per_block,
        schedule.n_warp,
        EXECUTION_MODES.index(schedule.execution_mode),
        schedule.dependence_protocol,
    )


def extract_workload_features(dag_successors, wavefront_list, argument_values,
                              function_props=None, flops_per_iteration=1,
                              thread_trip_counts=None, edges=None):
    """Features from host lists (reference interface) or, when
    ``dag_successors`` is an int, from counts the device inspector reports
    (``dag_successors`` = rows, ``wavefront_list`` = levels, ``edges``)."""
    if isinstance(dag_successors, (int, np.integer)):
        rows, levels = int(dag_successors), int(wavefront_list)
        edges = int(edges or 0)
    else:
        rows = len(dag_successors)
        edges = sum(len(successors) for successors in dag_successors)
        levels = len(wavefront_list)
    nonzeros = _nonzeros_from_pointer_arrays(argument_values, function_props)
    if nonzeros is None:
        nonzeros = rows + edges
    squares = 0
    if thread_trip_counts is None:
        work_items = invocations = 0
    elif isinstance(thread_trip_counts, dict):
        work_items = int(thread_trip_counts["work_items"])
        invocations = int(thread_trip_counts["invocations"])
        squares = int(thread_trip_counts.get("work_squares", 0))
    else:
        counts = tuple(max(int(c), 0) for c in thread_trip_counts)
        work_items, invocations = sum(counts), len(counts)
        squares = sum(c * c for c in counts)
    base = nonzeros if thread_trip_counts is None else work_items
    return WorkloadFeatures(
        rows=rows, edges=edges, levels=levels, nonzeros=nonzeros,
        flops=float(flops_per_iteration * base),
        memory_bytes=_array_bytes(argument_values),
        thread_work_items=work_items, thread_loop_invocations=invocations,
        thread_work_squares=squares)


# ---- trip counts of the thread-mapped loop -------------------------------

# Block iterations the host probe interprets at most; beyond, it visits an
# evenly strided sample and scales the totals (the ILU0 loop nest takes 3 us
# per row in CPython: 12 s for a 2048^2 grid, 0.2 s for the sample).
TRIP_PROBE_SAMPLE = 65536


def compile_thread_trip_counter(function_ast, thread_loop_iterator,
                                function_globals=None, block_iterator=None):
    """Host probe: the user function with the mapped loop replaced by the
    length of its range (side effects of the loop body removed).  Kept for
    interface parity; the decorator prefers :func:`segment_trip_counts`.
    With ``block_iterator`` the block loop's values pass through a hook that
    :func:`measure_thread_trip_counts` can use to sample them."""
    if thread_loop_iterator is None:
        return None
    module = deepcopy(function_ast)
    functions = [n for n in module.body if isinstance(n, ast.FunctionDef)]
    if len(functions) != 1:
        raise SchedulerError(
            "Thread-loop trip counting requires exactly one function.")
    function = functions[0]
    matches = []

    class Counter(ast.NodeTransformer):
        def visit_For(self, node):
            if not (isinstance(node.target, ast.Name)
                    and node.target.id == thread_loop_iterator):
                return self.generic_visit(node)
            matches.append(node)
            if node.orelse:
                raise SchedulerError(
                    "Thread-mapped loops with for/else cannot be trip-counted.")
            if not (isinstance(node.iter, ast.Call)
                    and isinstance(node.iter.func, ast.Name)
                    and node.iter.func.id == "range"
                    and not node.iter.keywords
                    and 1 <= len(node.iter.args) <= 3):
                raise SchedulerError(
                    "Thread-loop trip counting requires a range-based loop.")
            return ast.parse(
                f"_lcd_trip_counts.append(len({ast.unparse(node.iter)}))"
            ).body[0]

        def visit_Return(self, node):
            return ast.Return(
                value=ast.Name(id="_lcd_trip_counts", ctx=ast.Load()))

    class BlockValues(ast.NodeTransformer):
        def visit_For(self, node):
            self.generic_visit(node)
            if (isinstance(node.target, ast.Name)
                    and node.target.id == block_iterator):
                node.iter = ast.Call(
                    func=ast.Name(id="_lcd_block_values", ctx=ast.Load()),
                    args=[node.iter], keywords=[])
            return node

    function.body = [Counter().visit(s) for s in function.body]
    if block_iterator is not None:
        function.body = [BlockValues().visit(s) for s in function.body]
    flat = []
    for statement in function.body:
        flat.extend(statement if isinstance(statement, list) else [statement])
    function.body = flat
    if not matches:
        raise SchedulerError(
            f"Could not find thread-mapped loop {thread_loop_iterator!r}.")
    if len(matches) > 1:
        raise SchedulerError(
            "Thread-loop trip counting requires a unique loop iterator; "
            f"found {len(matches)} loops named {thread_loop_iterator!r}.")
    function.name = "_lcd_thread_trip_counter"
    function.decorator_list = []
    function.body.insert(0, ast.parse("_lcd_trip_counts = []").body[0])
    function.body.append(
        ast.Return(value=ast.Name(id="_lcd_trip_counts", ctx=ast.Load())))
    module.body = [function]
    namespace = dict(function_globals or {})
    namespace["_lcd_block_values"] = lambda values: values
    exec(compile(ast.fix_missing_locations(module),
                 "<lcd-thread-trip-counter>", "exec"), namespace)
    return namespace[function.name]


def measure_thread_trip_counts(counter, argument_values, argument_names,
                               sample_limit=None):
    """Run a trip-count probe on copies of the mutable arguments.  With
    ``sample_limit`` (and a probe compiled with its block iterator) a block
    loop over a longer ``range`` is visited with a stride and the totals are
    scaled; the result is then a dict of totals instead of the counts."""
    if counter is None:
        return None
    sampled = {"scale": 1.0}

    def block_values(values):
        if not isinstance(values, range) or len(values) <= sample_limit:
            return values
        taken = values[::-(-len(values) // sample_limit)]
        sampled["scale"] = len(values) / len(taken)
        return taken

    if sample_limit:
        counter.__globals__["_lcd_block_values"] = block_values
        try:
            counts = measure_thread_trip_counts(
                counter, argument_values, argument_names)
        finally:
            counter.__globals__["_lcd_block_values"] = lambda values: values
        if sampled["scale"] == 1.0:
            return counts
        trips = np.maximum(np.asarray(counts, dtype=np.int64), 0)
        scale = sampled["scale"]
        return {"work_items": int(round(float(trips.sum()) * scale)),
                "invocations": int(round(trips.size * scale)),
                "work_squares": int(round(float((trips * trips).sum())
                                          * scale))}
    arguments = []
    for name in argument_names:
        value = argument_values[name]
        if isinstance(value, np.ndarray):
            value = value.copy()
        elif isinstance(value, (list, dict, set)):
            value = deepcopy(value)
        arguments.append(value)
    return tuple(counter(*arguments))


def segment_trip_counts(thread_loop, block_iterator, argument_values):
    """Trip totals of ``for j in range(P[i] + a, P[i + 1] + b)`` directly
    from the pointer array (no interpretation of the user loop).  Returns
    ``None`` when the loop is not of that shape."""
    from lcd_amd.dependence import _split_offset

    if thread_loop is None or not (
            isinstance(thread_loop.iter, ast.Call)
            and len(thread_loop.iter.args) == 2):
        return None
    lower, lower_offset = _split_offset(thread_loop.iter.args[0])
    upper, upper_offset = _split_offset(thread_loop.iter.args[1])
    if not (isinstance(lower, ast.Subscript) and isinstance(upper, ast.Subscript)
            and isinstance(lower.value, ast.Name)
            and isinstance(upper.value, ast.Name)
            and lower.value.id == upper.value.id
            and isinstance(lower.slice, ast.Name)
            and lower.slice.id == block_iterator):
        return None
    base, one = _split_offset(upper.slice)
    if not (isinstance(base, ast.Name) and base.id == block_iterator
            and one == 1):
        return None
    pointers = argument_values.get(lower.value.id)
    if pointers is None:
        return None
    if hasattr(pointers, "copy_to_host"):
        pointers = pointers.copy_to_host()
    pointers = np.asarray(pointers, dtype=np.int64)
    trips = np.maximum(
        pointers[1:] + upper_offset - pointers[:-1] - lower_offset, 0)
    return {"work_items": int(trips.sum()), "invocations": int(trips.size),
            "work_squares": int((trips * trips).sum())}


def pointer_array_names(function_props):
    return [name for name, properties in (function_props or {}).items()
            if isinstance(name, str)
            and "monotonically_increasing" in properties]


def _nonzeros_from_pointer_arrays(argument_values, function_props):
    counts = []
    for name in pointer_array_names(function_props):
        value = argument_values.get(name)
        if value is None:
            continue
        if hasattr(value, "copy_to_host"):
            meta = value.shape
            if len(meta) == 1 and meta[0] >= 2:
                ends = value.copy_to_host()
                counts.append(int(ends[-1]) - int(ends[0]))
            continue
        pointers = np.asarray(value)
        if pointers.ndim == 1 and pointers.size >= 2:
            counts.append(int(pointers[-1]) - int(pointers[0]))
    return max(counts) if counts else None


def _array_bytes(argument_values):
    arrays = {}
    for value in argument_values.values():
        if isinstance(value, np.ndarray) or hasattr(value, "nbytes"):
            arrays[id(value)] = value
    return int(sum(array.nbytes for array in arrays.values()))


def count_inner_loop_flops(function_ast, block_iterator,
                           thread_loop_iterator=None):
    """Arithmetic operators in one iteration of the loop that the cost model
    prices (same result as compiler/scheduler.py:617-629): the thread-mapped
    loop when it is named and present, otherwise the most deeply nested
    ``for`` below the block loop; never less than 1."""
    block_loop = _loop_over(function_ast, block_iterator)
    if block_loop is None:
        return 1
    priced = None
    if thread_loop_iterator is not None:
        priced = _loop_over(block_loop, thread_loop_iterator)
    if priced is None:
        priced = _innermost_loop(block_loop)
    return max(sum(_arithmetic_ops(statement) for statement in priced.body), 1)


def _loop_over(tree, iterator):
    """First ``for <iterator> in ...`` of ``tree`` in breadth-first order."""
    return next((node for node in ast.walk(tree)
                 if isinstance(node, ast.For)
                 and isinstance(node.target, ast.Name)
                 and node.target.id == iterator), None)


def _innermost_loop(loop):
    """The ``for`` with the most enclosing loops below ``loop`` (``loop``
    itself when it has none); among equals the one nearest the root of the
    syntax tree, then the leftmost."""
    ranked = []

    def descend(node, loops, depth):
        for child in ast.iter_child_nodes(node):
            inside = loops + isinstance(child, ast.For)
            if isinstance(child, ast.For):
                ranked.append((-inside, depth + 1, len(ranked), child))
            descend(child, inside, depth + 1)

    descend(loop, 0, 0)
    return min(ranked)[3] if ranked else loop


def _arithmetic_ops(node):
    """Arithmetic operators that ``node`` executes once.  Index expressions
    of subscripts and the headers of nested loops are address and control
    work, not floating-point work, and are left out; an augmented assignment
    counts its operator and its right-hand side."""
    if isinstance(node, ast.Subscript):
        return _arithmetic_ops(node.value)
    if isinstance(node, ast.For):
        return sum(_arithmetic_ops(statement) for statement in node.body)
    if isinstance(node, ast.AugAssign):
        return (isinstance(node.op, ARITHMETIC_OPERATORS)
                + _arithmetic_ops(node.value))
    own = (isinstance(node, ast.BinOp)
           and isinstance(node.op, ARITHMETIC_OPERATORS))
    return own + sum(_arithmetic_ops(child)
                     for child in ast.iter_child_nodes(node))


# ---- plan cache keys -------------------------------------------------------

def inspection_fingerprint(values, content_names, device=None):
    """Cache key of one sparsity structure: content digests of the structure
    arrays plus dtype/shape of every array.  Host arrays are hashed on the
    host (128 bits, like the reference's blake2b-128); arrays already in HBM
    are digested on the device (``lcdhip_digest``)."""
    content = tuple((name, _value_digest(values.get(name), device))
                    for name in sorted(set(content_names)))
    shapes = []
    for name, value in sorted(values.items()):
        if isinstance(value, np.ndarray):
            shapes.append((name, value.dtype.str, value.shape))
        elif hasattr(value, "__cuda_array_interface__"):
            interface = value.__cuda_array_interface__
            shapes.append((name, interface["typestr"],
                           tuple(interface["shape"])))
    return content, tuple(shapes)


def _host_digest(data):
    """128-bit content digest of a host byte buffer.  The key only has to
    tell structures apart, so the fast non-cryptographic XXH3 is used when
    the module is there (about 10 GB/s against blake2b's 1.5: the 42 MB of a
    128^3 grid's structure arrays take 4 ms instead of 28 on every call);
    blake2b-128, the reference's choice, otherwise."""
    if _xxhash is not None:
        return _xxhash.xxh3_128_digest(data)
    return hashlib.blake2b(data, digest_size=16).digest()


def _value_digest(value, device=None):
    if hasattr(value, "__cuda_array_interface__"):
        if device is None:
            from lcd_amd import hip_runtime
            device = hip_runtime.default_device()
        interface = value.__cuda_array_interface__
        return (interface["typestr"], tuple(interface["shape"]),
                device.digest(value))
    if isinstance(value, np.ndarray):
        if value.dtype.hasobject:
            return object()
        contiguous = np.ascontiguousarray(value)
        return (contiguous.dtype.str, contiguous.shape,
                _host_digest(contiguous.reshape(-1).view(np.uint8)))
    if isinstance(value, (list, tuple)):
        try:
            return _value_digest(np.asarray(value), device)
        except (TypeError, ValueError):
            return object()
    if value is None or np.isscalar(value):
        return type(value).__name__, value
    return object()


def measure_arch_constants(device=None):
    """Machine constants measured on the GPU (``lcdhip_measure_arch``);
    data-sheet fallbacks when no device is present."""
    try:
        from lcd_amd import hip_runtime
        if device is None:
            if not hip_runtime.device_available():
                return FALLBACK_ARCH_CONSTANTS
            device = hip_runtime.default_device()
        measured = device.measure_arch()
    except Exception:
        return FALLBACK_ARCH_CONSTANTS
    return ArchConstants(**measured)

"""Expression and statement emission for the HIP lowering: the kernel ABI
names, the result record, kind inference (integer or double) and the emitter
that turns Python AST nodes of a loop body into HIP C++ text."""

import ast
from copy import deepcopy
from dataclasses import dataclass, field
import textwrap


class HIPLoweringError(Exception):
    """Base error for unsupported HIP lowering."""


class UnsupportedAtomicOperation(HIPLoweringError):
    """A reduction has no direct device atomic."""


COUNTER_DEPENDENCE = "counter"
PUSH_DEPENDENCE = "push"
PULL_DEPENDENCE = "pull"
MAILBOX_DEPENDENCE = "mailbox"
DEPENDENCE_PROTOCOLS = (COUNTER_DEPENDENCE, PUSH_DEPENDENCE, PULL_DEPENDENCE,
                        MAILBOX_DEPENDENCE)

HIP_EXECUTION_MODES = frozenset({"plain", "sync_free", "wavefront"})
WAVEFRONT_SIZE = 64
# Executor argument names: the kernel ABI the lowering and the runtime agree
# on (same names as compiler/cuda_lowering.py:51-64).
SYNC_FREE_ARGUMENTS = ("dep_count", "initial_dep_count", "dag_ptr", "dag_index",
                       "task_nodes", "task_ptr", "task_counter", "task_count")
PUSH_ARGUMENTS = ("dep_count", "initial_dep_count", "task_nodes", "task_ptr",
                  "task_counter", "task_count")
PULL_ARGUMENTS = ("done", "task_nodes", "task_ptr", "task_counter",
                  "task_count")
GATHER_ARGUMENTS = ("_lcd_in_ptr", "_lcd_in_pos", "_lcd_in_src",
                    "task_nodes", "task_ptr", "task_counter", "task_count")
VALUE_PULL_ARGUMENTS = ("task_nodes", "task_ptr", "task_counter", "task_count")
# level walker: the structure level-major from the inspector (task of (level,
# lane); source and operand position of its k-th incoming entry) and the
# number of levels
LEVEL_WALKER_ARGUMENTS = ("_lcd_lw_task", "_lcd_lw_src", "_lcd_lw_pos")
LEVEL_WALKER_LEVELS = "_lcd_lw_levels"
LEVEL_WALKER_TASKS = 4096      # tasks whose values fit the LDS copy
LEVEL_WALKER_ENTRIES = 4       # incoming entries per task the ring has room for
VALUE_WAIT_BEGIN = "//@lcd-wait-begin"
VALUE_WAIT_END = "//@lcd-wait-end"
MAILBOX_ARGUMENTS = ("_lcd_mailbox", "_lcd_in_ptr", "_lcd_out_slot",
                     "task_nodes", "task_ptr", "task_counter", "task_count")
WAVEFRONT_ARGUMENTS = ("task_nodes", "task_ptr", "band_start", "band_end")
STATUS_ARGUMENT = "_lcd_status"
HOST_LAUNCH_ARGUMENTS = frozenset({"band_ptr", "wavefront_ptr"})
INTEGER_EXECUTOR_ARRAYS = frozenset({
    "dep_count", "initial_dep_count", "dag_ptr", "dag_index", "task_nodes",
    "task_ptr", "task_counter", "done", STATUS_ARGUMENT, "_lcd_in_ptr",
    "_lcd_out_slot", "_lcd_in_pos", "_lcd_in_src",
    "_lcd_rec_in", "_lcd_rec_src", "_lcd_rec_pos",
})
# fixed-size records of the incoming listing in task order (tiled executor)
RECORD_ARGUMENTS = ("_lcd_rec_in", "_lcd_rec_src", "_lcd_rec_pos")
DEFAULT_SPIN_LIMIT = 1 << 22

_ATOMIC_CALLS = {"+": "lcd_atomic_add", "-": "lcd_atomic_sub",
                 "&": "lcd_atomic_and", "|": "lcd_atomic_or",
                 "^": "lcd_atomic_xor"}
_AUG_TEXT = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.Div: "/",
             ast.BitAnd: "&", ast.BitOr: "|", ast.BitXor: "^",
             ast.FloorDiv: "//", ast.Mod: "%"}
_BIN_TEXT = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.BitAnd: "&",
             ast.BitOr: "|", ast.BitXor: "^", ast.LShift: "<<",
             ast.RShift: ">>"}
_CMP_TEXT = {ast.Eq: "==", ast.NotEq: "!=", ast.Lt: "<", ast.LtE: "<=",
             ast.Gt: ">", ast.GtE: ">="}
INT = "int"
FLOAT = "float"


@dataclass
class HIPLoweringResult:
    """Everything the runtime needs to compile, bind and launch one variant.

    Field names follow CUDALoweringResult (compiler/cuda_lowering.py:72-98).
    ``source`` is HIP C++; ``launcher_source`` is the Python launcher.
    """

    source: str
    kernel_source: str
    launcher_source: str
    launcher_ast: ast.Module
    kernel_name: str
    launcher_name: str
    reset_kernel_name: str | None
    kernel_arguments: list
    launcher_arguments: list
    lifted_variables: list
    lifted_loop_parameters: list
    host_prelude: list
    host_epilogue: list
    atomic_statement_ids: set
    execution_mode: str
    auxiliary_arguments: list
    thread_loop_iterator: str | None = None
    thread_unroll_factor: int = 1
    host_loop_iterators: tuple = ()
    n_warp: int | None = None
    warp_mapped: bool = False
    dependence_protocol: str = COUNTER_DEPENDENCE
    task_lanes: int = 1
    threads_per_block: int = 128
    tasks_per_block: int = 128
    array_arguments: dict = field(default_factory=dict)   # name -> INT|FLOAT
    scalar_arguments: dict = field(default_factory=dict)  # name -> INT|FLOAT
    written_arrays: tuple = ()
    zero_initialised: dict = field(default_factory=dict)  # lifted -> shape src
    persistent: bool = False
    function_name: str = ""
    mailbox_index_array: str | None = None
    # pull protocol without flags: consumers poll the producers' elements of
    # this array, which the reset kernel fills with the empty marker
    value_flag_array: str | None = None
    # tiled executor whose LDS copy and flag array are indexed by the place
    # of a task in the queue (tiles that do not follow the ids)
    tile_by_position: bool = False
    # one wavefront runs the tasks in program order (chain-like DAGs whose
    # edges span fewer than 64 iterations)
    band_walker: bool = False
    # one wavefront takes a level per step (small DAGs with narrow levels):
    # the incoming entries per task it has room for, or 0
    level_walker: int = 0
    # grid sweep (lcd_amd/hip_grid_sweep.py): its geometry, the names of the
    # staging kernels (matrix part, other part, solution back to its array),
    # whether anything is staged per launch, the arrays the matrix part reads
    # and the launcher function that stages the matrix part
    grid_sweep: dict | None = None
    stage_kernels: tuple = ()
    sweep_dynamic: bool = False
    stage_static_arrays: tuple = ()
    restage_launcher_name: str | None = None
    # level launches read operands laid out in level order (staging kernels
    # ``stage_kernels``; sources named by their place in the level order)
    level_records: bool = False
    # the pointer array of the task's own segment (ILU0's row), and whether
    # that segment is kept in registers (segments of at most 64 entries)
    segment_pointer: str | None = None
    segment_registers: bool = False
    # tables of structure searches keyed by the task's own positions:
    # ("at", name, lookup table, index array) = lookup[index[p]] by p;
    # ("pair", "_lcd_pair", pointer array, index array) with "_lcd_pair_base":
    # byte offsets; ("start", "_lcd_pair_start", pointer array, index array) =
    # pointer[index[p]] by p
    structure_tables: tuple = ()
    # lifted zero-initialised arrays the executor needs no host-side clear for
    executor_initialised: tuple = ()
    # kernel that gathers position-indexed operands into consumer order at
    # the start of every launch (gathered mailbox), and its argument names
    task_record_lanes: int | None = None
    queue_node_loads: tuple = ()     # (argument, structure array, offset)
    published_array: str | None = None   # its final values go to _lcd_pub
    stage_kernel_name: str | None = None
    stage_kernel_arguments: tuple = ()
    # tiled persistent executor: block-iterator values per tile, or None
    tile_rows: int | None = None
    spin_limit: int = DEFAULT_SPIN_LIMIT   # watchdog limit the caller chose
    # time budget of one launch of a persistent executor in seconds: None =
    # from the depth and size of the DAG, 0 = none (the poll count still ends
    # a wait that cannot end)
    watchdog_seconds: float | None = None

    @property
    def module_source(self):
        return self.source


# --------------------------------------------------------------------------
# small AST helpers

def _names_in(node):
    return {n.id for n in ast.walk(node) if isinstance(n, ast.Name)}


def _stored_names(statements):
    names = []
    for statement in statements:
        for node in ast.walk(statement):
            if (isinstance(node, ast.Name) and isinstance(node.ctx, ast.Store)
                    and node.id not in names):
                names.append(node.id)
    return names


def _is_range_loop(node):
    return (isinstance(node, ast.For) and isinstance(node.target, ast.Name)
            and isinstance(node.iter, ast.Call)
            and isinstance(node.iter.func, ast.Name)
            and node.iter.func.id == "range" and not node.iter.keywords
            and 1 <= len(node.iter.args) <= 3 and not node.orelse)


def _to_module(code):
    if isinstance(code, ast.Module):
        return deepcopy(code)
    if isinstance(code, ast.FunctionDef):
        return ast.Module(body=[deepcopy(code)], type_ignores=[])
    if isinstance(code, str):
        return ast.parse(textwrap.dedent(code))
    raise HIPLoweringError("HIP lowering expects source text or an AST.")


def _normalize_mode(execution_mode):
    mode = execution_mode.replace("-", "_")
    if mode not in HIP_EXECUTION_MODES:
        raise HIPLoweringError(
            f"Unknown HIP execution mode {execution_mode!r}; expected one of "
            f"{sorted(HIP_EXECUTION_MODES)}.")
    return mode


def _normalize_reductions(reductions):
    """Accept a DependenceAnalysis, a dict/list of reduction sites, or
    ``(lineno, col)`` tuples."""
    if reductions is None:
        return {}
    if hasattr(reductions, "reductions"):
        reductions = reductions.reductions
    if isinstance(reductions, dict):
        reductions = reductions.values()
    sites = {}
    for position, site in enumerate(reductions):
        if isinstance(site, tuple) and len(site) == 2:
            sites[site] = (f"S{position + 1}", None)
            continue
        location = getattr(site, "location", None)
        if location is None or getattr(site, "statement_id", None) is None:
            raise HIPLoweringError(
                "Reduction metadata must come from dependence analysis and "
                "contain a source location, statement ID, and operator.")
        sites[tuple(location)] = (site.statement_id, site.operator)
    return sites


# --------------------------------------------------------------------------
# type inference

class _Kinds:
    """INT/FLOAT kinds of arrays, scalars and locals, inferred from use."""

    def __init__(self, function, function_props, lookup_names, forced=None):
        self.function = function
        arguments = [a.arg for a in function.args.args]
        subscripted = {
            n.value.id for n in ast.walk(function)
            if isinstance(n, ast.Subscript) and isinstance(n.value, ast.Name)}
        demanded = set(lookup_names)
        for key in (function_props or {}):
            for name in (key if isinstance(key, tuple) else (key,)):
                if isinstance(name, str):
                    demanded.add(name)
        index_contexts = []
        for node in ast.walk(function):
            if isinstance(node, ast.Subscript):
                index_contexts.append(node.slice)
            if (isinstance(node, ast.Call) and isinstance(node.func, ast.Name)
                    and node.func.id == "range"):
                index_contexts.extend(node.args)
        for context in index_contexts:
            demanded |= _names_in(context)
        assignments = [
            (node.targets[0].id, node.value) for node in ast.walk(function)
            if isinstance(node, ast.Assign) and len(node.targets) == 1
            and isinstance(node.targets[0], ast.Name)]
        changed = True
        while changed:
            changed = False
            for name, value in assignments:
                if name in demanded:
                    if isinstance(value, ast.Call):
                        continue  # e.g. x = np.zeros(n): x stays a value array
                    new = _names_in(value) - demanded
                    if new:
                        demanded |= new
                        changed = True
        self.arrays = {}
        for name in subscripted | set(lookup_names):
            self.arrays[name] = INT if name in demanded else FLOAT
        for name in INTEGER_EXECUTOR_ARRAYS:
            self.arrays[name] = INT
        self.arrays["_lcd_mailbox"] = FLOAT
        for name, kind in (forced or {}).items():
            if name in self.arrays:
                self.arrays[name] = kind
        self.scalars = {
            name: (INT if name in demanded else FLOAT)
            for name in arguments if name not in subscripted}
        self.locals = {}
        self.iterators = {
            node.target.id for node in ast.walk(function)
            if isinstance(node, ast.For) and isinstance(node.target, ast.Name)}

    def infer_locals(self, statements, extra_int=()):
        names = _stored_names(statements)
        for name in names:
            self.locals.setdefault(name, INT)
        for name in extra_int:
            self.locals[name] = INT
        changed = True
        while changed:
            changed = False
            for statement in statements:
                for node in ast.walk(statement):
                    target, value = None, None
                    if (isinstance(node, ast.Assign) and len(node.targets) == 1
                            and isinstance(node.targets[0], ast.Name)):
                        target, value = node.targets[0].id, node.value
                    elif (isinstance(node, ast.AugAssign)
                          and isinstance(node.target, ast.Name)):
                        target = node.target.id
                        value = ast.BinOp(left=ast.Name(id=target, ctx=ast.Load()),
                                          op=node.op, right=node.value)
                    if target is None or target in self.iterators:
                        continue
                    if self.kind(value) == FLOAT and self.locals.get(target) != FLOAT:
                        self.locals[target] = FLOAT
                        changed = True

    def kind(self, node):
        if isinstance(node, ast.Constant):
            return FLOAT if isinstance(node.value, float) else INT
        if isinstance(node, ast.Name):
            if node.id in self.iterators:
                return INT
            if node.id in self.locals:
                return self.locals[node.id]
            return self.scalars.get(node.id, INT)
        if isinstance(node, ast.Subscript):
            if isinstance(node.value, ast.Name):
                return self.arrays.get(node.value.id, FLOAT)
            return FLOAT
        if isinstance(node, ast.BinOp):
            if isinstance(node.op, (ast.Div, ast.Pow)):
                return FLOAT
            kinds = (self.kind(node.left), self.kind(node.right))
            return FLOAT if FLOAT in kinds else INT
        if isinstance(node, ast.UnaryOp):
            return INT if isinstance(node.op, ast.Not) else self.kind(node.operand)
        if isinstance(node, (ast.Compare, ast.BoolOp)):
            return INT
        if isinstance(node, ast.IfExp):
            kinds = (self.kind(node.body), self.kind(node.orelse))
            return FLOAT if FLOAT in kinds else INT
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Name):
            if node.func.id in ("float",):
                return FLOAT
            if node.func.id in ("int", "len", "_lcd_sorted_find",
                                "_lcd_rseg_first", "_lcd_pair_at"):
                return INT
            if node.func.id in ("abs", "min", "max"):
                kinds = [self.kind(a) for a in node.args]
                return FLOAT if FLOAT in kinds else INT
        return FLOAT


# --------------------------------------------------------------------------
# Python AST -> C++ text

class _Emitter:
    def __init__(self, kinds, reductions, lowered_ids, coherent_arrays=()):
        self.kinds = kinds
        self.reductions = reductions
        self.lowered_ids = lowered_ids
        # arrays other tasks write while this kernel runs: every access goes
        # through device-scope (cache-bypassing / write-through) accessors
        self.coherent_arrays = set(coherent_arrays)
        self.mailbox = None
        self.lowerer = None
        self.segment = None     # own-segment staging plan (HIPLowerer)
        self.published = None   # final values published to a flagged buffer
        self.tile = None        # tiled executor plan (HIPLowerer)
        self.in_mapped = None   # iterator of the distributed loop being emitted

    def _register_position(self, index):
        """How a position of the own segment kept in registers is reached:
        'lane' for the distributed loop's own iterator inside that loop
        (lane l works on entry l), 'uniform' for a loop variable that walks
        the segment in the task's uniform code, None for anything else."""
        segment = self.segment
        if not (isinstance(index, ast.Name) and index.id in segment["owned"]):
            return None
        if self.in_mapped is None:
            return "uniform"
        return "lane" if self.in_mapped == index.id else None

    # ---- expressions
    def expr(self, node):
        k = self.kinds
        if isinstance(node, ast.Constant):
            if isinstance(node.value, bool):
                return "1" if node.value else "0"
            if isinstance(node.value, int):
                return str(node.value)
            if isinstance(node.value, float):
                return repr(node.value)
            raise HIPLoweringError(f"Unsupported constant {node.value!r}.")
        if isinstance(node, ast.Name):
            return node.id
        if isinstance(node, ast.Subscript):
            if not isinstance(node.value, ast.Name):
                raise HIPLoweringError("Only 1-D array indexing is supported.")
            element = f"{node.value.id}[{self.expr(node.slice)}]"
            segment = self.segment
            if (segment is not None and node.value.id == segment["array"]
                    and segment.get("registers")):
                place = self._register_position(node.slice)
                if place == "lane":
                    return "_lcd_rseg"
                if place == "uniform":
                    return (f"lcd_rseg_uni(_lcd_rseg, {node.slice.id} - "
                            "_lcd_seg_base)")
                if segment.get("foreign") and self.published.get("plain"):
                    return element
                if segment.get("foreign"):
                    # (never a position of the task's own segment)
                    return (f"lcd_pub_ldp(_lcd_pub, {self.expr(node.slice)}, "
                            f"{STATUS_ARGUMENT}, _task_aborted, _lcd_t0, "
                            "_lcd_ptile, _lcd_tpos0, _lcd_tlen)")
                return ("lcd_rseg_ldp(_lcd_pub, _lcd_seg, _lcd_seg_base, "
                        f"_lcd_seg_own, {self.expr(node.slice)}, "
                        f"{STATUS_ARGUMENT}, _task_aborted, _lcd_t0, "
                        "_lcd_ptile, _lcd_tpos0, _lcd_tlen)")
            if (segment is not None and node.value.id == segment["array"]
                    and self.published is not None):
                return (f"lcd_seg_ldp({node.value.id}, _lcd_pub, _lcd_seg, "
                        "_lcd_seg_base, _lcd_seg_limit, _lcd_seg_own, "
                        f"{self.expr(node.slice)}, {STATUS_ARGUMENT}, "
                        "_task_aborted, _lcd_t0, _lcd_ptile, _lcd_tpos0, "
                        "_lcd_tlen)")
            if segment is not None and node.value.id == segment["array"]:
                name = ("lcd_seg_ldc" if node.value.id in self.coherent_arrays
                        else "lcd_seg_ld")
                return (f"{name}({node.value.id}, _lcd_seg, _lcd_seg_base, "
                        f"_lcd_seg_limit, {self.expr(node.slice)})")
            if self.tile is not None and node.value.id == self.tile["array"]:
                return self.tile_load(self.expr(node.slice))
            if node.value.id in self.coherent_arrays:
                return f"lcd_ld(&{element})"
            return element
        if isinstance(node, ast.BinOp):
            left, right = self.expr(node.left), self.expr(node.right)
            if isinstance(node.op, ast.Div):
                if k.kind(node.left) == INT:
                    left = f"(double)({left})"
                if k.kind(node.right) == INT:
                    right = f"(double)({right})"
                return f"({left} / {right})"
            if isinstance(node.op, ast.FloorDiv):
                if k.kind(node) == INT:
                    return f"lcd_floordiv({left}, {right})"
                return f"floor({left} / {right})"
            if isinstance(node.op, ast.Mod):
                if k.kind(node) == INT:
                    return f"lcd_mod({left}, {right})"
                return f"lcd_fmod({left}, {right})"
            if isinstance(node.op, ast.Pow):
                return f"pow((double)({left}), (double)({right}))"
            text = _BIN_TEXT.get(type(node.op))
            if text is None:
                raise HIPLoweringError(
                    f"Unsupported operator {type(node.op).__name__}.")
            return f"({left} {text} {right})"
        if isinstance(node, ast.UnaryOp):
            operand = self.expr(node.operand)
            if isinstance(node.op, ast.USub):
                return f"(-{operand})"
            if isinstance(node.op, ast.UAdd):
                return operand
            if isinstance(node.op, ast.Not):
                return f"(!{operand})"
            if isinstance(node.op, ast.Invert):
                return f"(~{operand})"
        if isinstance(node, ast.Compare):
            parts = []
            left = node.left
            for op, right in zip(node.ops, node.comparators):
                text = _CMP_TEXT.get(type(op))
                if text is None:
                    raise HIPLoweringError(
                        f"Unsupported comparison {type(op).__name__}.")
                parts.append(f"({self.expr(left)} {text} {self.expr(right)})")
                left = right
            return parts[0] if len(parts) == 1 else "(" + " && ".join(parts) + ")"
        if isinstance(node, ast.BoolOp):
            joiner = " && " if isinstance(node.op, ast.And) else " || "
            return "(" + joiner.join(self.expr(v) for v in node.values) + ")"
        if isinstance(node, ast.IfExp):
            return (f"({self.expr(node.test)} ? {self.expr(node.body)} : "
                    f"{self.expr(node.orelse)})")
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Name):
            name = node.func.id
            args = [self.expr(a) for a in node.args]
            if name == "abs" and len(args) == 1:
                return (f"fabs({args[0]})" if k.kind(node.args[0]) == FLOAT
                        else f"lcd_iabs({args[0]})")
            if name in ("min", "max") and len(args) == 2:
                if FLOAT in (k.kind(node.args[0]), k.kind(node.args[1])):
                    return f"f{name}((double)({args[0]}), (double)({args[1]}))"
                return f"lcd_i{name}({args[0]}, {args[1]})"
            if name == "float" and len(args) == 1:
                return f"(double)({args[0]})"
            if name == "int" and len(args) == 1:
                return f"(lcd_index_t)({args[0]})"
            if name == "_lcd_sorted_find" and len(args) == 4:
                return f"lcd_sorted_find({', '.join(args)})"
            if name == "_lcd_rseg_first" and len(args) == 1:
                return f"lcd_rseg_first({args[0]}, _lcd_seg_base)"
            if name == "_lcd_wdiv" and len(args) == 2:
                # (band walker) a division whose divisor was known ahead
                return f"_lcd_wdiv({args[0]}, {args[1]}, _lcd_wr)"
            if name == "_lcd_pair_at" and len(args) == 2:
                return (f"lcd_pair_pos(_lcd_pair[_lcd_pair_row + (({args[0]}) - "
                        f"_lcd_seg_base) * _lcd_seg_own + (({args[1]}) - "
                        f"_lcd_seg_base)], _lcd_pair_start[{args[0]}])")
            if (name == "_lcd_raw" and self.published is not None
                    and self.segment.get("registers")):
                target = node.args[0]
                if self.segment.get("foreign") and self.published.get("plain"):
                    return self.element(target)
                if self.segment.get("foreign"):
                    return ("lcd_pub_ld(_lcd_pub, _lcd_ptile, _lcd_tpos0, "
                            f"_lcd_tlen, {self.expr(target.slice)})")
                return ("lcd_rseg_ldr(_lcd_pub, _lcd_seg, _lcd_seg_base, "
                        f"_lcd_seg_own, {self.expr(target.slice)}, _lcd_ptile, "
                        "_lcd_tpos0, _lcd_tlen)")
            if name == "_lcd_raw" and self.published is not None:
                target = node.args[0]
                return (f"lcd_seg_ldr({target.value.id}, _lcd_pub, _lcd_seg, "
                        "_lcd_seg_base, _lcd_seg_limit, _lcd_seg_own, "
                        f"{self.expr(target.slice)}, _lcd_ptile, _lcd_tpos0, "
                        "_lcd_tlen)")
            if name == "_lcd_pdiv":
                return f"lcd_pdiv({args[0]}, {args[1]}, _lcd_rcp)"
            if name == "_lcd_settle" and self.published is not None:
                target = node.args[0]
                if (self.segment is not None and self.segment.get("foreign")
                        and self.published.get("plain")):
                    return args[1]
                if self.segment is not None and self.segment.get("foreign"):
                    return (f"lcd_pull_settle(_lcd_pub, "
                            f"{self.expr(target.slice)}, {args[1]}, "
                            f"{STATUS_ARGUMENT}, _task_aborted, _lcd_t0, "
                            "_lcd_ptile, _lcd_tpos0, _lcd_tlen)")
                return ("lcd_seg_settle(_lcd_pub, _lcd_seg_base, _lcd_seg_own, "
                        f"{self.expr(target.slice)}, {args[1]}, "
                        f"{STATUS_ARGUMENT}, _task_aborted, _lcd_t0, "
                        "_lcd_ptile, _lcd_tpos0, _lcd_tlen)")
        raise HIPLoweringError(
            f"Unsupported expression in a device loop: {ast.unparse(node)!r}.")

    def element(self, target):
        """``X[e]`` as an lvalue (no accessor)."""
        if not (isinstance(target, ast.Subscript)
                and isinstance(target.value, ast.Name)):
            raise HIPLoweringError("Only 1-D array indexing is supported.")
        return f"{target.value.id}[{self.expr(target.slice)}]"

    def tile_load(self, index_text):
        """Read of the value-flagged array: LDS inside the running tile."""
        array = self.tile["array"]
        if self.tile.get("by_position"):
            raise HIPLoweringError(
                "Tiles addressed by queue position serve tasks that read "
                f"{array} through the incoming listing only.")
        return (f"lcd_tile_ld({array}, _lcd_tile, _lcd_tile_row0, "
                f"_lcd_tile_rows, {index_text})")

    def store(self, target, value_text):
        element = self.element(target)
        if (self.tile is not None and target.value.id == self.tile["array"]
                and self.tile.get("by_position")):
            # the flag copy (LDS slot and memory) is indexed by the task's
            # place in the queue; the array itself gets a plain store
            if self.expr(target.slice) != self.lowerer.loop_iterator:
                raise HIPLoweringError(
                    "Tiles addressed by queue position need tasks that "
                    f"write their own element of {target.value.id} only.")
            return ("{ lcd_tile_st(_lcd_xq, _lcd_tile, _lcd_tile_row0, "
                    f"_lcd_tile_rows, (lcd_index_t)_task, {value_text}); "
                    f"{element} = {value_text}; }}")
        level = getattr(self.lowerer, "_level_records", None)
        if (level is not None and self.mailbox is not None
                and target.value.id == self.mailbox["array"]):
            # level launches over operands in level order: the consumers
            # read the copy of the array in that order
            return (f"{{ _lcd_xq[_task] = {value_text}; "
                    f"{element} = {value_text}; }}")
        if self.tile is not None and target.value.id == self.tile["array"]:
            return (f"lcd_tile_st({target.value.id}, _lcd_tile, _lcd_tile_row0, "
                    f"_lcd_tile_rows, {self.expr(target.slice)}, {value_text});")
        segment = self.segment
        if (segment is not None and target.value.id == segment["array"]
                and segment.get("registers")):
            place = self._register_position(target.slice)
            offset = f"{self.expr(target.slice)} - _lcd_seg_base"
            if place == "lane":
                if segment.get("foreign"):
                    return f"_lcd_rseg = {value_text};"
                return (f"{{ _lcd_rseg = {value_text}; "
                        f"_lcd_seg[{offset}] = _lcd_rseg; }}")
            if place == "uniform":
                if segment.get("foreign"):
                    return (f"if ((lcd_index_t)(threadIdx.x & 63u) == {offset}) "
                            f"_lcd_rseg = {value_text};")
                return (f"lcd_rseg_put(_lcd_rseg, _lcd_seg, {offset}, "
                        f"{value_text});")
            raise HIPLoweringError(
                "A segment kept in registers is written through the loop "
                f"variables that walk it; got {ast.unparse(target)!r}.")
        if segment is not None and target.value.id == segment["array"]:
            name = ("lcd_seg_stc" if target.value.id in self.coherent_arrays
                    else "lcd_seg_st")
            return (f"{name}({target.value.id}, _lcd_seg, _lcd_seg_base, "
                    f"_lcd_seg_limit, {self.expr(target.slice)}, {value_text});")
        if target.value.id in self.coherent_arrays:
            return f"lcd_st(&{element}, {value_text});"
        return f"{element} = {value_text};"

    # ---- statements
    def block(self, statements, indent, hooks=None):
        lines = []
        for statement in statements:
            lines.extend(self.stmt(statement, indent, hooks))
        return lines

    def range_parts(self, loop):
        args = loop.iter.args
        if len(args) == 1:
            return "0", self.expr(args[0]), "1"
        if len(args) == 2:
            return self.expr(args[0]), self.expr(args[1]), "1"
        return self.expr(args[0]), self.expr(args[1]), self.expr(args[2])

    def atomic(self, node):
        location = (getattr(node, "lineno", None), getattr(node, "col_offset", None))
        site = self.reductions.get(location)
        if site is None:
            return None
        statement_id, operator = site
        operator = operator or _AUG_TEXT.get(type(node.op))
        call = _ATOMIC_CALLS.get(operator)
        if call is None:
            raise UnsupportedAtomicOperation(
                f"Reduction {statement_id} uses {operator!r}, which has no "
                "direct atomic lowering in this stage.")
        if not (isinstance(node.target, ast.Subscript)
                and isinstance(node.target.value, ast.Name)):
            raise HIPLoweringError(
                "Device atomics require an indexed 1-D array target.")
        self.lowered_ids.add(statement_id)
        atomic = f"{call}(&{self.element(node.target)}, {self.expr(node.value)});"
        box = self.mailbox
        if box is not None and node.target.value.id == box["array"]:
            # one message per position instead of an atomic update; the
            # consumer adds the messages in source order
            value = self.expr(node.value)
            if operator == "-":
                value = f"(-({value}))"
            slot = self.expr(box["slot"])
            store = f"lcd_st(&_lcd_mailbox[{slot}], {value});"
            guard = self.lowerer.mailbox_guard_text()
            if guard is None:
                return store
            return f"if ({guard}) {store} else {atomic}"
        return atomic

    def stmt(self, node, indent, hooks=None):
        pad = "    " * indent
        if isinstance(node, ast.Pass):
            return []
        if isinstance(node, ast.Expr):
            if isinstance(node.value, ast.Constant):
                return []
            raise HIPLoweringError(
                f"Unsupported statement {ast.unparse(node)!r}.")
        if isinstance(node, ast.Assign):
            if len(node.targets) != 1:
                raise HIPLoweringError("Chained assignment is not supported.")
            target = node.targets[0]
            if isinstance(target, ast.Subscript):
                return [pad + self.store(target, self.expr(node.value))]
            if isinstance(target, ast.Name):
                return [f"{pad}{target.id} = {self.expr(node.value)};"]
            raise HIPLoweringError("Unsupported assignment target.")
        if isinstance(node, ast.AugAssign):
            atomic = self.atomic(node)
            if atomic is not None:
                return [pad + atomic]
            expanded = ast.BinOp(left=deepcopy(node.target), op=node.op,
                                 right=node.value)
            for sub in ast.walk(expanded.left):
                if hasattr(sub, "ctx"):
                    sub.ctx = ast.Load()
            if isinstance(node.target, ast.Subscript):
                return [pad + self.store(node.target, self.expr(expanded))]
            return [f"{pad}{node.target.id} = {self.expr(expanded)};"]
        if isinstance(node, ast.If):
            lines = [f"{pad}if ({self.expr(node.test)}) {{"]
            lines += self.block(node.body, indent + 1, hooks)
            if node.orelse:
                lines.append(f"{pad}}} else {{")
                lines += self.block(node.orelse, indent + 1, hooks)
            lines.append(f"{pad}}}")
            return lines
        if isinstance(node, ast.While):
            lines = [f"{pad}while ({self.expr(node.test)}) {{"]
            lines += self.block(node.body, indent + 1, hooks)
            lines.append(f"{pad}}}")
            return lines
        if isinstance(node, ast.Break):
            return [f"{pad}break;"]
        if isinstance(node, ast.Continue):
            return [f"{pad}continue;"]
        if isinstance(node, ast.For):
            if hooks is not None and hooks.is_mapped(node):
                return hooks.mapped_loop(node, indent)
            if not _is_range_loop(node):
                raise HIPLoweringError(
                    "Device loops must be `for name in range(...)`.")
            lower, upper, step = self.range_parts(node)
            name = node.target.id
            if step == "1":
                head = (f"{pad}for ({name} = {lower}; {name} < {upper}; "
                        f"++{name}) {{")
            else:
                head = (f"{pad}for ({name} = {lower}; lcd_in_range({name}, "
                        f"{upper}, {step}); {name} += {step}) {{")
            return [head, *self.block(node.body, indent + 1, hooks), f"{pad}}}"]
        raise HIPLoweringError(
            f"Unsupported statement in a device loop: {ast.unparse(node)!r}.")


# --------------------------------------------------------------------------
# the lowerer


class _MappedLoopHooks:
    """Turns the thread-mapped loop into a lane-strided loop."""

    def __init__(self, lowerer, emitter, loop):
        self.lowerer = lowerer
        self.emitter = emitter
        self.loop = loop
        self.partials = []   # (partial_name, target_node, op)
        self.value_pull = None

    def is_mapped(self, node):
        return node is self.loop

    def mapped_loop(self, node, indent):
        low = self.lowerer
        pad = "    " * indent
        emitter = self.emitter
        lower, upper, step = emitter.range_parts(node)
        if step != "1":
            raise HIPLoweringError(
                "The thread-mapped loop must have a unit step.")
        name = node.target.id
        lanes = "LCD_TASK_LANES"
        unroll = low.thread_unroll_factor
        body = deepcopy(node.body)
        # lanes only need a group fence after the loop when it stored to
        # memory that later uniform code may read (atomics and register
        # partial sums do not)
        stores = any(
            isinstance(sub, (ast.Assign, ast.AugAssign))
            and any(isinstance(t, ast.Subscript) for t in (
                sub.targets if isinstance(sub, ast.Assign) else [sub.target]))
            and (getattr(sub, "lineno", None), getattr(sub, "col_offset", None))
            not in low.reductions
            for statement in node.body for sub in ast.walk(statement))
        lines = []
        for partial, _, _ in self.partials:
            lines.append(f"{pad}{partial} = 0.0;")
        if self.value_pull is not None:
            return self._value_pull_loop(node, body, indent, lines, stores)
        registers = (emitter.segment is not None
                     and emitter.segment.get("registers")
                     and name in emitter.segment["owned"])
        emitter.in_mapped = name
        try:
            body_lines = emitter.block(
                body, indent + (2 if unroll > 1 else 1), None)
        finally:
            emitter.in_mapped = None
        hook_lines = low.push_hook_lines(indent + (2 if unroll > 1 else 1))
        if registers:
            # lane l works on entry l of the segment (at most 64 entries:
            # one trip), so the entry a lane updates is its own register
            if unroll != 1 or low._first_iteration_reload:
                raise HIPLoweringError(
                    "A segment in registers needs the plain distributed loop.")
            lines.append(f"{pad}{name} = lcd_rseg_first({lower}, _lcd_seg_base);")
            lines.append(f"{pad}if ({name} < {upper}) {{")
            lines += body_lines + hook_lines
            lines.append(f"{pad}}}")
            # (register updates need no fence)
            return lines + self._after_loop(pad, False)
        if unroll == 1:
            lines.append(f"{pad}for ({name} = ({lower}) + _lane; {name} < {upper}; "
                         f"{name} += {lanes}) {{")
            lines += [f"{pad}    {line}" for line in low._first_iteration_reload]
            lines += body_lines + hook_lines
            lines.append(f"{pad}}}")
        else:
            base = f"_{name}_base"
            lines.append(f"{pad}for (lcd_index_t {base} = ({lower}) + _lane; "
                         f"{base} < {upper}; {base} += {lanes} * {unroll}) {{")
            lines.append(f"{pad}#pragma unroll")
            lines.append(f"{pad}    for (int _u = 0; _u < {unroll}; ++_u) {{")
            lines.append(f"{pad}        {name} = {base} + _u * {lanes};")
            lines.append(f"{pad}        if ({name} < {upper}) {{")
            lines += ["    " + line for line in body_lines + hook_lines]
            lines.append(f"{pad}        }}")
            lines.append(f"{pad}    }}")
            lines.append(f"{pad}}}")
        lines += self._after_loop(pad, stores)
        return lines

    def _value_pull_loop(self, node, body, indent, lines, stores):
        """The distributed loop of a value-flagged pull: resumable.  Each lane
        walks its positions as far as the producers' values are final (not
        the empty marker) and keeps its position across polls; the lines
        between the two markers are re-entered by the executor's poll loop."""
        low, emitter = self.lowerer, self.emitter
        pad = "    " * indent
        plan = self.value_pull
        lower, upper, _ = emitter.range_parts(node)
        name = node.target.id
        array = plan["array"]
        endpoint = (low._hook_endpoint if low._hook_endpoint is not None
                    else low.direct_dependence.endpoint)
        guard = (low._hook_guard if low._hook_endpoint is not None
                 else low.direct_dependence.guard)
        endpoint_texts = {plan["endpoint_text"], ast.unparse(endpoint)}

        class Substitute(ast.NodeTransformer):
            count = 0

            def visit_Subscript(self, sub):
                if (isinstance(sub.value, ast.Name) and sub.value.id == array
                        and ast.unparse(sub.slice) in endpoint_texts):
                    Substitute.count += 1
                    return ast.copy_location(
                        ast.Name(id="_lcd_vf", ctx=ast.Load()), sub)
                return self.generic_visit(sub)

        body = [Substitute().visit(statement) for statement in body]
        if Substitute.count == 0:
            raise HIPLoweringError(
                "Value-flagged pull found no read of the producers' values.")
        low._kinds.locals["_lcd_vf"] = FLOAT
        body_lines = emitter.block(body, indent + 1, None)
        lines.append(f"{pad}{name} = ({lower}) + _lane;")
        reload = list(low._first_iteration_reload)
        first = f"if ({name} != ({lower}) + _lane) {{"
        if len(reload) == 1 and reload[0].startswith(first):
            # the entries of a position stay in their registers across polls:
            # they are fetched again only for a new position
            low._kinds.locals["_lcd_vat"] = INT
            if "_lcd_vat" not in low._extra_locals:
                low._extra_locals.append("_lcd_vat")
            lines.append(f"{pad}_lcd_vat = {name};")
            reload = [f"if ({name} != _lcd_vat) {{ _lcd_vat = {name};"
                      + reload[0][len(first):]]
        lines.append(VALUE_WAIT_BEGIN)
        lines.append(f"{pad}for (; {name} < {upper}; {name} += LCD_TASK_LANES) {{")
        lines += [f"{pad}    {line}" for line in reload]
        load = (emitter.tile_load(emitter.expr(endpoint))
                if emitter.tile is not None and emitter.tile["array"] == array
                else f"{low.pull_load}(&{array}[{emitter.expr(endpoint)}])")
        lines.append(f"{pad}    double _lcd_vf = {load};")
        if guard is None:
            lines.append(f"{pad}    if (lcd_is_empty(_lcd_vf)) break;")
        else:
            # a read the DAG does not order sees the initial zero
            lines.append(f"{pad}    if (lcd_is_empty(_lcd_vf)) {{ "
                         f"if ({emitter.expr(guard)}) break; _lcd_vf = 0.0; }}")
        lines += body_lines
        lines.append(f"{pad}}}")
        lines.append(VALUE_WAIT_END)
        plan["remaining"] = f"{name} < {upper}"
        lines += self._after_loop(pad, stores)
        return lines

    def _after_loop(self, pad, stores):
        low, emitter = self.lowerer, self.emitter
        lines = []
        if stores:
            lines.append(f"{pad}{low.group_sync}")
        for partial, target, op in self.partials:
            total = low.group_total(partial)
            op_text = "+" if isinstance(op, ast.Add) else "-"
            target_text = emitter.expr(target)
            lines.append(f"{pad}{partial} = {total};")
            if isinstance(target, ast.Subscript):
                lines.append(f"{pad}if (_lane == 0) " + emitter.store(
                    target, f"{target_text} {op_text} {partial}"))
                lines.append(f"{pad}{low.group_sync}")
            else:
                lines.append(f"{pad}{target_text} = {target_text} {op_text} {partial};")
        return lines

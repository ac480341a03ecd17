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
from dataclasses import dataclass, field
import textwrap

from lcd_amd.dependence import _split_offset
from lcd_amd.structural_lookups import (
    match_segment_search,
    structure_aliases,
    rewrite_structural_lookups,
    segmented_array_pairs,
    structural_lookup_names,
)


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
INT, FLOAT = "int", "float"


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
            if node.func.id in ("int", "len", "_lcd_sorted_find"):
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
                    and self.published is not None):
                return (f"lcd_seg_ldp({node.value.id}, _lcd_pub, _lcd_seg, "
                        "_lcd_seg_base, _lcd_seg_limit, _lcd_seg_own, "
                        f"{self.expr(node.slice)}, {STATUS_ARGUMENT}, "
                        "_task_aborted)")
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
            if name == "_lcd_raw" and self.published is not None:
                target = node.args[0]
                return (f"lcd_seg_ldr({target.value.id}, _lcd_pub, _lcd_seg, "
                        "_lcd_seg_base, _lcd_seg_limit, _lcd_seg_own, "
                        f"{self.expr(target.slice)})")
            if name == "_lcd_settle" and self.published is not None:
                target = node.args[0]
                return ("lcd_seg_settle(_lcd_pub, _lcd_seg_base, _lcd_seg_own, "
                        f"{self.expr(target.slice)}, {args[1]}, "
                        f"{STATUS_ARGUMENT}, _task_aborted)")
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
        return (f"lcd_tile_ld({array}, _lcd_tile, _lcd_tile_row0, "
                f"_lcd_tile_rows, {index_text})")

    def store(self, target, value_text):
        element = self.element(target)
        if self.tile is not None and target.value.id == self.tile["array"]:
            return (f"lcd_tile_st({target.value.id}, _lcd_tile, _lcd_tile_row0, "
                    f"_lcd_tile_rows, {self.expr(target.slice)}, {value_text});")
        segment = self.segment
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

_PRELUDE = r"""
// ---- generated by lcd_amd.hip_lowering for gfx950 -------------------------
// (hiprtc provides the HIP device headers implicitly)
typedef LCD_INDEX_TYPE lcd_index_t;
#define LCD_AGENT __HIP_MEMORY_SCOPE_AGENT

__device__ __forceinline__ lcd_index_t lcd_floordiv(lcd_index_t a, lcd_index_t b) {
    lcd_index_t q = a / b;
    return ((a % b != 0) && ((a < 0) != (b < 0))) ? q - 1 : q;
}
__device__ __forceinline__ lcd_index_t lcd_mod(lcd_index_t a, lcd_index_t b) {
    lcd_index_t r = a % b;
    return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}
__device__ __forceinline__ double lcd_fmod(double a, double b) {
    double r = fmod(a, b);
    return (r != 0.0 && ((r < 0.0) != (b < 0.0))) ? r + b : r;
}
__device__ __forceinline__ lcd_index_t lcd_iabs(lcd_index_t a) { return a < 0 ? -a : a; }
__device__ __forceinline__ lcd_index_t lcd_imin(lcd_index_t a, lcd_index_t b) { return a < b ? a : b; }
__device__ __forceinline__ lcd_index_t lcd_imax(lcd_index_t a, lcd_index_t b) { return a > b ? a : b; }
__device__ __forceinline__ bool lcd_in_range(lcd_index_t v, lcd_index_t stop, lcd_index_t step) {
    return step > 0 ? v < stop : v > stop;
}
// First position p in [lo, hi) of a sorted segment with idx[p] == key, else -1.
template <class T>
__device__ __forceinline__ lcd_index_t lcd_sorted_find(const T* idx, lcd_index_t lo,
                                                       lcd_index_t hi, lcd_index_t key) {
    if (hi - lo <= 16 && hi > lo) {
        // short segment: sixteen independent loads (one memory round trip)
        // instead of a chain of dependent probes
        lcd_index_t found = (lcd_index_t)-1;
#pragma unroll
        for (int t = 15; t >= 0; --t) {
            const lcd_index_t p = lo + t < hi ? lo + t : hi - 1;
            if ((lcd_index_t)idx[p] == key) found = p;
        }
        return found;
    }
    lcd_index_t left = lo, right = hi;
    while (left < right) {
        lcd_index_t middle = (left + right) >> 1;
        if ((lcd_index_t)idx[middle] < key) left = middle + 1; else right = middle;
    }
    return (left < hi && (lcd_index_t)idx[left] == key) ? left : (lcd_index_t)-1;
}
// A task's own segment of an array it updates in place, staged in LDS: an
// access inside [base, base + limit) goes to the staged copy, any other
// position to memory (limit == 0 switches the staging off).
template <class T>
__device__ __forceinline__ T lcd_seg_ld(const T* x, const T* seg, lcd_index_t base,
                                        lcd_index_t limit, lcd_index_t p) {
    const unsigned off = (unsigned)(p - base);
    return off < (unsigned)limit ? seg[off] : x[p];
}
template <class T, class V>
__device__ __forceinline__ void lcd_seg_st(T* x, T* seg, lcd_index_t base,
                                           lcd_index_t limit, lcd_index_t p, V v) {
    const unsigned off = (unsigned)(p - base);
    if (off < (unsigned)limit) seg[off] = (T)v; else x[p] = (T)v;
}
// Device-scope relaxed atomics (fp64 add is a hardware L2 atomic on CDNA3/4).
template <class T, class V> __device__ __forceinline__ void lcd_atomic_add(T* p, V v) {
    __hip_atomic_fetch_add(p, (T)v, __ATOMIC_RELAXED, LCD_AGENT);
}
template <class T, class V> __device__ __forceinline__ void lcd_atomic_sub(T* p, V v) {
    __hip_atomic_fetch_add(p, (T)(-(T)v), __ATOMIC_RELAXED, LCD_AGENT);
}
template <class T, class V> __device__ __forceinline__ void lcd_atomic_and(T* p, V v) {
    __hip_atomic_fetch_and(p, (T)v, __ATOMIC_RELAXED, LCD_AGENT);
}
template <class T, class V> __device__ __forceinline__ void lcd_atomic_or(T* p, V v) {
    __hip_atomic_fetch_or(p, (T)v, __ATOMIC_RELAXED, LCD_AGENT);
}
template <class T, class V> __device__ __forceinline__ void lcd_atomic_xor(T* p, V v) {
    __hip_atomic_fetch_xor(p, (T)v, __ATOMIC_RELAXED, LCD_AGENT);
}
__device__ __forceinline__ int lcd_load_relaxed(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, LCD_AGENT);
}
// Coherent accessors for arrays that other tasks write while the kernel runs
// (sync-free executors).  Device-scope relaxed atomics: loads always observe
// the device coherence point, stores are written through to it, so no L2
// write-back or invalidation is ever needed around a dependence hand-off.
template <class T> __device__ __forceinline__ T lcd_ld(const T* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, LCD_AGENT);
}
template <class T, class V> __device__ __forceinline__ void lcd_st(T* p, V v) {
    __hip_atomic_store(p, (T)v, __ATOMIC_RELAXED, LCD_AGENT);
}
template <class T>
__device__ __forceinline__ T lcd_seg_ldc(const T* x, const T* seg, lcd_index_t base,
                                         lcd_index_t limit, lcd_index_t p) {
    const unsigned off = (unsigned)(p - base);
    return off < (unsigned)limit ? seg[off] : lcd_ld(&x[p]);
}
template <class T, class V>
__device__ __forceinline__ void lcd_seg_stc(T* x, T* seg, lcd_index_t base,
                                            lcd_index_t limit, lcd_index_t p, V v) {
    const unsigned off = (unsigned)(p - base);
    if (off < (unsigned)limit) seg[off] = (T)v; else lcd_st(&x[p], v);
}
// Mailbox protocol: a slot holds this quiet-NaN bit pattern until its message
// (a finite product) has been stored; both 32-bit halves are equal so a
// 32-bit fill resets the buffer.
#define LCD_EMPTY_WORD 0x7FF84C43u
__device__ __forceinline__ bool lcd_is_empty(double v) {
    return __double_as_longlong(v) == (long long)0x7FF84C437FF84C43ull;
}
// An element stored once per launch over the empty marker: any other value a
// load returns is final whichever cache served it, so only the marker itself
// has to be confirmed by a coherent load.
__device__ __forceinline__ double lcd_ld_once(const double* p) {
    double v = *p;
    if (lcd_is_empty(v)) v = lcd_ld(p);
    return v;
}
// Published values: a task works on its own segment (staged in LDS, or in
// place when it does not fit) and ends by storing the final values to a
// buffer that started as the empty marker; a read of another task's element
// polls that buffer.  With one task per wavefront in queue order the poll may
// block: the producer sits earlier in the queue and waits for nobody behind.
__device__ __forceinline__ double lcd_pull_settle(const double* pub, lcd_index_t p,
                                                  double v, int* status, bool& aborted) {
    if (!lcd_is_empty(v) || aborted) return v;
    unsigned spins = 0;
    while (lcd_is_empty(v)) {
#if LCD_SPIN_SLEEP > 0
        __builtin_amdgcn_s_sleep(LCD_SPIN_SLEEP);
#endif
        v = lcd_ld(&pub[p]);
        if ((++spins & 1023u) == 0u && (spins > (unsigned)LCD_SPIN_LIMIT
                                        || lcd_load_relaxed(status) != 0)) {
            status[0] = 1;
            aborted = true;
            break;
        }
    }
    return v;
}
// first attempt only: the load is in flight while the task does other work
__device__ __forceinline__ double lcd_seg_ldr(const double* x, const double* pub,
                                              const double* seg, lcd_index_t base,
                                              lcd_index_t limit, lcd_index_t own,
                                              lcd_index_t p) {
    const unsigned off = (unsigned)(p - base);
    if (off < (unsigned)limit) return seg[off];
    // one load instruction for both arrays: two in exclusive branches made
    // the compiler wait for everything in flight where the branches meet
    return lcd_ld(off < (unsigned)own ? &x[p] : &pub[p]);
}
// ... and the wait for it where the value is used
__device__ __forceinline__ double lcd_seg_settle(const double* pub, lcd_index_t base,
                                                 lcd_index_t own, lcd_index_t p,
                                                 double v, int* status, bool& aborted) {
    const unsigned off = (unsigned)(p - base);
    return off < (unsigned)own ? v : lcd_pull_settle(pub, p, v, status, aborted);
}
__device__ __forceinline__ double lcd_seg_ldp(const double* x, const double* pub,
                                              const double* seg, lcd_index_t base,
                                              lcd_index_t limit, lcd_index_t own,
                                              lcd_index_t p, int* status, bool& aborted) {
    const unsigned off = (unsigned)(p - base);
    if (off < (unsigned)limit) return seg[off];
    const double v = lcd_ld(off < (unsigned)own ? &x[p] : &pub[p]);
    return off < (unsigned)own ? v : lcd_pull_settle(pub, p, v, status, aborted);
}
__device__ __forceinline__ double lcd_empty() {
    return __longlong_as_double((long long)0x7FF84C437FF84C43ull);
}
// Tiled executor: the elements [row0, row0 + rows) of the value-flagged array
// live in LDS while their tile runs.  A read inside the tile polls LDS (the
// producer is a wavefront of this workgroup), any other read the device
// coherence point; a task's final store goes to both.
template <class T>
__device__ __forceinline__ T lcd_tile_ld(const T* x, const T* tile, lcd_index_t row0,
                                         lcd_index_t rows, lcd_index_t p) {
    const unsigned off = (unsigned)(p - row0);
    if (off < (unsigned)rows)
        return __hip_atomic_load(&tile[off], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    return lcd_ld(&x[p]);
}
template <class T, class V>
__device__ __forceinline__ void lcd_tile_st(T* x, T* tile, lcd_index_t row0,
                                            lcd_index_t rows, lcd_index_t p, V v) {
    const unsigned off = (unsigned)(p - row0);
    if (off < (unsigned)rows)
        __hip_atomic_store(&tile[off], (T)v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
    lcd_st(&x[p], v);
}
// Lane k of every group of four adjacent lanes, to all four (one DPP move per
// 32-bit half instead of a cross-lane permute through LDS).
template <int K>
__device__ __forceinline__ double lcd_quad_broadcast(double v) {
    const int ctrl = K | (K << 2) | (K << 4) | (K << 6);   // quad_perm [K,K,K,K]
    const long long bits = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_mov_dpp((int)bits, ctrl, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(bits >> 32), ctrl, 0xf, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}
// True when no lane of the task group raises the flag (one ballot instead of
// a butterfly of shuffles; lanes of other groups that are masked off read 0).
__device__ __forceinline__ bool lcd_group_none(bool flag) {
    const unsigned long long raised = __ballot(flag);
#if LCD_TASK_LANES >= 64
    return raised == 0ull;
#else
    const int shift = (int)((threadIdx.x & 63) / LCD_TASK_LANES) * LCD_TASK_LANES;
    return ((raised >> shift) & ((1ull << LCD_TASK_LANES) - 1ull)) == 0ull;
#endif
}
// Release: every store/atomic this wavefront issued has completed at the
// coherence point before anything after the fence is issued.
__device__ __forceinline__ void lcd_release_fence() {
#ifdef LCD_FULL_FENCES
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
}
// Between a task's atomic updates of other tasks' elements and the counter
// decrement that releases them.  The updates are device-scope atomics, which
// are performed at the device coherence point (never left dirty in an L2), so
// it is enough to wait until they have completed: no L2 write-back is needed.
__device__ __forceinline__ void lcd_push_fence() {
#ifdef LCD_FULL_FENCES
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#endif
}
// Acquire: the ready test is a completed device-scope load and the GPU issues
// nothing speculatively past the branch on it; with coherent accessors for
// the data, only the compiler has to be kept from hoisting loads.
__device__ __forceinline__ void lcd_acquire_fence() {
#ifdef LCD_FULL_FENCES
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#else
    asm volatile("" ::: "memory");
#endif
}
// Sum over the LCD_TASK_LANES lanes of one task group (xor butterfly: every
// lane ends with the total, the compiler lowers the fixed masks to DPP).
__device__ __forceinline__ double lcd_group_sum(double v) {
#if LCD_TASK_LANES <= 64
#pragma unroll
    for (int offset = LCD_TASK_LANES / 2; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, LCD_TASK_LANES);
#endif
    return v;
}
"""

_GROUP_SYNC_WAVE = ("__builtin_amdgcn_fence(__ATOMIC_ACQ_REL, \"wavefront\"); "
                    "__builtin_amdgcn_wave_barrier();")
_GROUP_SYNC_BLOCK = "__syncthreads();"


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
        body_lines = emitter.block(body, indent + (2 if unroll > 1 else 1), None)
        hook_lines = low.push_hook_lines(indent + (2 if unroll > 1 else 1))
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
        lines.append(VALUE_WAIT_BEGIN)
        lines.append(f"{pad}for (; {name} < {upper}; {name} += LCD_TASK_LANES) {{")
        lines += [f"{pad}    {line}" for line in low._first_iteration_reload]
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


class HIPLowerer:
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
                 publish_values=True, look_ahead=True, segment_capacity=None):
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
        self.dependence_protocol = (
            dependence_protocol
            if (direct_dependence is not None
                and direct_dependence.kind == required_kind
                and self.warp_mapped and self.execution_mode == "sync_free"
                and sync_free_ready_count == 0)
            else COUNTER_DEPENDENCE)
        self._mailbox = None
        self.group_sync = (_GROUP_SYNC_BLOCK if self.block_task
                           else _GROUP_SYNC_WAVE)
        self.segmented_sorted = segmented_array_pairs(self.function_props)

    # ---- mailbox protocol
    def _mailbox_plan(self, body):
        """The mailbox protocol applies when the loop's only cross-task
        writes are ``X[endpoint] +=/-= value`` inside the top level of the
        distributed loop, the endpoint is the push dependence's, and the task
        reads and rewrites its own ``X[i]`` at the top level."""
        dependence = self.direct_dependence
        endpoint = dependence.endpoint
        if not (isinstance(endpoint, ast.Subscript)
                and isinstance(endpoint.value, ast.Name)):
            return None
        mapped = self._find_mapped_loop(body)
        if mapped is None or mapped not in body:
            return None
        sites = [node for statement in body for node in ast.walk(statement)
                 if isinstance(node, ast.AugAssign)
                 and (node.lineno, node.col_offset) in self.reductions]
        if not sites or len(sites) != len(self.reductions):
            return None
        arrays = set()
        for site in sites:
            if site not in mapped.body:
                return None
            if not isinstance(site.op, (ast.Add, ast.Sub)):
                return None
            if not (isinstance(site.target, ast.Subscript)
                    and isinstance(site.target.value, ast.Name)
                    and ast.unparse(site.target.slice) == ast.unparse(endpoint)):
                return None
            arrays.add(site.target.value.id)
        if len(arrays) != 1:
            return None
        array = arrays.pop()
        own_text = f"{array}[{self.loop_iterator}]"
        rewritten = False
        for statement in body:
            if statement is mapped:
                continue
            if (isinstance(statement, ast.Assign) and len(statement.targets) == 1
                    and ast.unparse(statement.targets[0]) == own_text
                    and any(ast.unparse(n) == own_text
                            for n in ast.walk(statement.value)
                            if isinstance(n, ast.Subscript))):
                rewritten = True
        if not rewritten:
            return None
        return {"array": array, "position": deepcopy(endpoint.slice),
                "index_array": endpoint.value.id, "own_text": own_text,
                "sites": sites, "mapped": mapped, "gather": None}

    def _fully_rewritten_arrays(self, body, target_loop, zero_initialised):
        """Lifted ``X = np.zeros(count)`` arrays whose element ``X[i]`` every
        task assigns unconditionally at its top level, with ``i`` running over
        ``range(count)``: after the loop no element keeps its initial zero."""
        arguments = target_loop.iter.args
        if len(arguments) != 1:
            return set()
        count = ast.unparse(arguments[0])
        found = set()
        for name, shape in zero_initialised.items():
            if shape != count:
                continue
            own_text = f"{name}[{self.loop_iterator}]"
            if any(isinstance(statement, ast.Assign)
                   and len(statement.targets) == 1
                   and ast.unparse(statement.targets[0]) == own_text
                   for statement in body):
                found.add(name)
        return found

    def _value_pull_plan(self, body):
        """The pull protocol can drop its ``done`` flags when the values
        themselves tell whether they are final: the consumers read
        ``X[endpoint]`` only inside the distributed loop, ``X`` is a lifted
        zero-initialised array every task writes exactly once (its own
        element, kept in a register until the end of the task), and nothing
        else is written.  ``X`` then starts as the empty marker and a consumer
        advances through its loop as far as final values are there."""
        dependence = self.direct_dependence
        if (dependence is None or self.block_task or self.chain_tasks
                or self.thread_unroll_factor != 1
                or not self.promote_own_elements
                or not self.prefetch_node_loads):
            return None
        mapped = self._find_mapped_loop(body)
        if mapped is None or mapped not in body or len(mapped.iter.args) != 2:
            return None
        endpoint_text = ast.unparse(dependence.endpoint)
        arrays = {
            node.value.id for statement in mapped.body
            for node in ast.walk(statement)
            if isinstance(node, ast.Subscript)
            and isinstance(node.value, ast.Name)
            and isinstance(node.ctx, ast.Load)
            and node.value.id in self._all_written
            and ast.unparse(node.slice) == endpoint_text}
        if len(arrays) != 1 or self._all_written != arrays:
            return None
        array = next(iter(arrays))
        if array not in self._fully_rewritten:
            return None
        # inside the distributed loop X is read at the endpoint only; its
        # other accesses are the task's own element (a privatised reduction)
        for statement in mapped.body:
            for node in ast.walk(statement):
                if not (isinstance(node, ast.Subscript)
                        and isinstance(node.value, ast.Name)
                        and node.value.id == array):
                    continue
                index = ast.unparse(node.slice)
                if index == self.loop_iterator:
                    continue
                if not isinstance(node.ctx, ast.Load) or index != endpoint_text:
                    return None
        return {"array": array, "endpoint_text": endpoint_text}

    def _sequential_pull_plan(self, body):
        """Pull protocol for a task whose producers are enumerated by one of
        its own sequential loops (ILU0-CSR: ``for k_ptr in <row>: k =
        A_indices[k_ptr]; if k >= i: break; ...``): instead of waiting until
        every producer is done and then running the whole body, the loop is
        made resumable and waits for producer ``k`` at the top of iteration
        ``k_ptr``.  The work on early pivots overlaps the wait for the late
        ones; what stays on the critical path is the last pivots' work.
        9-point grid 1024^2: 35.4 ms (counters) -> 18.2 ms, against 23.1 ms
        for level launches."""
        dependence = self.direct_dependence
        if (self.execution_mode != "sync_free" or self.block_task
                or self.chain_tasks or dependence.iterator is None):
            return None
        loops = [statement for statement in body
                 if isinstance(statement, ast.For)
                 and isinstance(statement.target, ast.Name)
                 and statement.target.id == dependence.iterator]
        if len(loops) != 1 or not _is_range_loop(loops[0]) or (
                len(loops[0].iter.args) != 2):
            return None
        loop = loops[0]
        # the loop must be the rule's: same bounds once aliases are resolved
        aliases = structure_aliases(ast.Module(body=body, type_ignores=[]))
        expected = dependence.thread_loop.iter.args
        for bound, wanted in zip(loop.iter.args, expected):
            resolved = aliases.get(bound.id, bound) if isinstance(
                bound, ast.Name) else bound
            if ast.unparse(resolved) != ast.unparse(wanted):
                return None
        # the wait goes after the statements that leave the loop at the
        # task's own entry (`if k >= i: break`)
        split = 0
        for position, statement in enumerate(loop.body):
            if (isinstance(statement, ast.If) and len(statement.body) == 1
                    and isinstance(statement.body[0], ast.Break)
                    and not statement.orelse):
                split = position + 1
                break
        for statement in loop.body[:split]:
            for node in ast.walk(statement):
                if isinstance(node, ast.Subscript) and isinstance(
                        node.value, ast.Name) and (
                            node.value.id in self._all_written):
                    return None          # reads a producer before the wait
        return {"iterator": dependence.iterator,
                "endpoint": dependence.endpoint, "remaining": "_lcd_blocked"}

    def _gather_plan(self, box, arguments, lifted_loop_parameters):
        """Gathered form of the mailbox protocol: no message slots at all.

        When the distributed loop holds nothing but the one reduction
        ``X[endpoint] op= value`` and ``value`` is a function of read-only
        data at the position, the producer's block iterator and the
        producer's final own element ``X[i]``, the consumer can form the
        product itself: it walks its incoming positions (``_lcd_in_pos``,
        ``_lcd_in_src``), polls ``X[source]`` -- ``X`` starts as the empty
        marker and is written once per task, so the value is the flag -- and
        adds the products in (source, position) order.  The producer's loop
        disappears; a task ends with the single store of its own element.
        Position-indexed operands (``Ax[j]``) are gathered into consumer
        order by a staging kernel at the start of every launch.  On the 128^3
        7-point grid: 0.71 ms against 0.75 ms with message slots, and the
        form the tiled executor needs (0.60 ms)."""
        mapped, sites = box["mapped"], box["sites"]
        array = box["array"]
        if (len(sites) != 1 or mapped.body != [sites[0]]
                or self._all_written != {array} or self.block_task
                or not self.promote_own_elements):
            return None
        site = sites[0]
        kinds = self._kinds
        readonly = {name for name in kinds.arrays
                    if name not in self._all_written}
        scalars = {name for name in arguments if name not in kinds.arrays}
        scalars |= set(lifted_loop_parameters)
        position, owner = mapped.target.id, self.loop_iterator
        for node in ast.walk(site.value):
            if isinstance(node, ast.Call):
                return None
            if isinstance(node, ast.Subscript):
                if not isinstance(node.value, ast.Name):
                    return None
                if node.value.id == array:
                    if ast.unparse(node.slice) != owner:
                        return None
                elif node.value.id not in readonly:
                    return None
            elif isinstance(node, ast.Name):
                if node.id not in ({position, owner, array} | readonly
                                   | scalars):
                    return None

        class Substitute(ast.NodeTransformer):
            def visit_Subscript(self, node):
                if (isinstance(node.value, ast.Name)
                        and node.value.id == array):
                    return ast.Name(id="_g_value", ctx=ast.Load())
                return self.generic_visit(node)

            def visit_Name(self, node):
                if node.id == position:
                    return ast.Name(id="_g_pos", ctx=node.ctx)
                if node.id == owner:
                    return ast.Name(id="_g_src", ctx=node.ctx)
                return node

        value = ast.fix_missing_locations(
            Substitute().visit(deepcopy(site.value)))
        # operands that do not wait for the producer load ahead of the poll
        operands = []

        class Operands(ast.NodeTransformer):
            def visit_Subscript(self, node):
                node = self.generic_visit(node)
                if (isinstance(node.value, ast.Name)
                        and node.value.id in readonly):
                    name = f"_g_operand_{len(operands)}"
                    operands.append((name, deepcopy(node),
                                     kinds.arrays.get(node.value.id, FLOAT)))
                    return ast.Name(id=name, ctx=ast.Load())
                return node

        value = ast.fix_missing_locations(Operands().visit(value))
        for name, _, kind in operands:
            kinds.locals[name] = kind
        kinds.locals["_g_value"] = FLOAT
        kinds.locals["_g_pos"] = INT
        kinds.locals["_g_src"] = INT
        # operands indexed by the position only are gathered into consumer
        # order by a staging kernel at the start of every launch, so the
        # executor reads them contiguously (an `Ax[in_pos[s]]` gather is a
        # second dependent, scattered load in front of every task)
        staged = {}
        if self.stage_operands:
            for name, node, kind in operands:
                names = _names_in(node.slice)
                if "_g_pos" in names and "_g_src" not in names:
                    staged[name] = f"_lcd_staged_{len(staged)}"
                    kinds.arrays[staged[name]] = kind
        needs_position = any(
            "_g_pos" in _names_in(node.slice) for name, node, _ in operands
            if name not in staged) or "_g_pos" in _names_in(value)
        return {"value": value, "operands": operands, "staged": staged,
                "needs_position": needs_position,
                "negate": isinstance(site.op, ast.Sub)}

    def _mailbox_slot_load(self):
        """``_lcd_out_slot[position]``: the message slot a position writes."""
        return ast.fix_missing_locations(ast.Subscript(
            value=ast.Name(id="_lcd_out_slot", ctx=ast.Load()),
            slice=deepcopy(self._mailbox["position"]), ctx=ast.Load()))

    def mailbox_guard_text(self):
        dependence = self.direct_dependence
        guard = (self._hook_guard if self._hook_endpoint is not None
                 else dependence.guard)
        return None if guard is None else self._emitter.expr(guard)

    # ---- helpers used by the hooks
    def group_total(self, partial):
        if self.block_task:
            return f"lcd_block_sum({partial}, _lcd_reduce)"
        if self.task_lanes == 1:
            return partial
        return f"lcd_group_sum({partial})"

    def push_hook_lines(self, indent):
        if self.dependence_protocol != PUSH_DEPENDENCE:
            return []
        pad = "    " * indent
        dependence = self.direct_dependence
        endpoint_node = self._hook_endpoint or dependence.endpoint
        guard_node = (self._hook_guard if self._hook_endpoint is not None
                      else dependence.guard)
        endpoint = self._emitter.expr(endpoint_node)
        lines = [f"{pad}lcd_push_fence();"]
        if guard_node is not None:
            lines.append(f"{pad}if ({self._emitter.expr(guard_node)})")
            lines.append(f"{pad}    lcd_atomic_sub(&dep_count[{endpoint}], 1);")
        else:
            lines.append(f"{pad}lcd_atomic_sub(&dep_count[{endpoint}], 1);")
        return lines

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
                self.dependence_protocol = PUSH_DEPENDENCE
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
        if self._mailbox is not None and (
                self._mailbox["array"] in self._fully_rewritten):
            self._own_zero_arrays.add(self._mailbox["array"])
            if self.gather_messages and self.value_flags:
                self._mailbox["gather"] = self._gather_plan(
                    self._mailbox, arguments, lifted_loop_parameters)
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
                               "buffer": "_lcd_pub"}
            kinds.arrays["_lcd_pub"] = FLOAT
        if self.tile_rows:
            self._tile = self._tile_plan(target_loop)
        if (self.task_records and self._mailbox is not None
                and self._mailbox["gather"] is not None):
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
        emitter = _Emitter(kinds, self.reductions, lowered_ids,
                           coherent_arrays=coherent)
        emitter.segment = self._segment
        emitter.published = self._published
        emitter.tile = self._tile
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
        missing = ({sid for sid, _ in self.reductions.values()} - lowered_ids)
        if missing:
            raise HIPLoweringError(
                "Reduction statements were not found in the selected loop: "
                + ", ".join(sorted(missing)))

        function_name = function.name
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
            queue_node_loads=tuple(self._queue_node_loads),
            published_array=(self._published["array"]
                             if self._published else None),
            task_record_lanes=(
                self.task_lanes if self._mailbox
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
            elif self.dependence_protocol == MAILBOX_DEPENDENCE:
                names = list(MAILBOX_ARGUMENTS)
            else:
                names = list(SYNC_FREE_ARGUMENTS)
            return names + [STATUS_ARGUMENT]
        if self.execution_mode == "wavefront":
            return list(WAVEFRONT_ARGUMENTS)
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

    def _privatize(self, loop, hooks, outer_assigned):
        """Updates of group-invariant targets inside the mapped loop become
        per-lane partial sums (compiler/cuda_lowering.py:2061-2121)."""
        loop_local = {loop.target.id} | set(_stored_names(loop.body))
        safe = True
        counter = [0]

        def invariant(target):
            if isinstance(target, ast.Name):
                return target.id in outer_assigned
            if isinstance(target, ast.Subscript):
                return not (_names_in(target) & loop_local)
            return False

        lowerer = self

        class Privatizer(ast.NodeTransformer):
            depth = 0

            def visit_AugAssign(self, node):
                location = (node.lineno, node.col_offset)
                if location in lowerer.reductions or not invariant(node.target):
                    return self.generic_visit(node)
                if not isinstance(node.op, (ast.Add, ast.Sub)):
                    nonlocal safe
                    safe = False
                    return node
                name = f"_thread_partial_{counter[0]}"
                counter[0] += 1
                hooks.partials.append((name, deepcopy(node.target), node.op))
                return ast.copy_location(ast.AugAssign(
                    target=ast.Name(id=name, ctx=ast.Store()), op=ast.Add(),
                    value=node.value), node)

            def visit_Assign(self, node):
                nonlocal safe
                if any(invariant(t) for t in node.targets):
                    safe = False
                return node

            def visit_For(self, node):
                self.depth += 1
                node = self.generic_visit(node)
                self.depth -= 1
                return node

            visit_While = visit_For

            def visit_Break(self, node):
                nonlocal safe
                if self.depth == 0:
                    safe = False
                return node

            visit_Continue = visit_Break

        loop.body = [Privatizer().visit(s) for s in loop.body]
        ast.fix_missing_locations(loop)
        return safe

    def _tile_plan(self, target_loop):
        """Tiled persistent executor: one workgroup runs the tasks of
        ``tile_rows`` consecutive block-iterator values (a tile) and keeps
        their elements of the value-flagged array in LDS, so that hand-offs
        between tasks of a tile are LDS round trips between wavefronts of one
        workgroup; only edges that cross tiles pay the device-scope hop.
        Needs a protocol in which the value is the flag (value-flagged pull
        or the gathered mailbox), node ids 0 .. n-1 in topological order (a
        tile then depends on lower tiles only, whatever the tile size) and
        wavefront-sized tasks; other combinations keep the flat queue
        (``tile_rows`` of the result is then None)."""
        rows = self.tile_rows
        if not isinstance(rows, int) or rows <= 0 or rows * 8 > 65536:
            raise HIPLoweringError(
                "tile_rows must be a positive integer of at most 8192 "
                "(64 KB of LDS).")
        array = None
        if self._value_pull is not None:
            array = self._value_pull["array"]
        elif self._mailbox is not None and self._mailbox["gather"] is not None:
            array = self._mailbox["array"]
        if (array is None or self.execution_mode != "sync_free"
                or self.block_task or len(target_loop.iter.args) != 1):
            return None      # the flat queue serves every other combination
        return {"array": array, "rows": rows}

    def _segment_plan(self, body, arguments):
        """In-place updates of the task's own segment ``X[P[i] .. P[i+1])``
        (ILU0 rewrites row ``i`` once per pivot) are staged in LDS: the
        segment is read once, updated there, and written back at the end of
        the task, instead of a store -> load round trip through memory per
        update.  Applies when ``X`` is written at positions walked by loops
        over ``range(P[i] + a, P[i + 1] - b)`` and is no reduction target;
        accesses are dispatched at run time (inside the staged range or not),
        so reads of other tasks' segments keep going to memory."""
        kinds = self._kinds
        written = self._all_written
        reduced = set()
        for statement in body:
            for node in ast.walk(statement):
                if (isinstance(node, ast.AugAssign)
                        and (node.lineno, node.col_offset) in self.reductions
                        and isinstance(node.target, ast.Subscript)
                        and isinstance(node.target.value, ast.Name)):
                    reduced.add(node.target.value.id)
        aliases = {}
        for statement in body:
            if (isinstance(statement, ast.Assign) and len(statement.targets) == 1
                    and isinstance(statement.targets[0], ast.Name)):
                name = statement.targets[0].id
                aliases[name] = None if name in aliases else statement.value
        it = self.loop_iterator

        def pointer_of(node, offset):
            """``P`` if the node is ``P[i + offset]`` (+/- a constant that
            keeps it inside the segment), through one alias."""
            if isinstance(node, ast.Name) and aliases.get(node.id) is not None:
                node = aliases[node.id]
            if isinstance(node, ast.BinOp) and isinstance(
                    node.right, ast.Constant) and isinstance(
                        node.right.value, int):
                inward = ast.Add if offset == 0 else ast.Sub
                if isinstance(node.op, inward) and node.right.value >= 0:
                    return pointer_of(node.left, offset)
                return None
            if not (isinstance(node, ast.Subscript)
                    and isinstance(node.value, ast.Name)
                    and node.value.id not in written
                    and kinds.arrays.get(node.value.id) == INT):
                return None
            want = it if offset == 0 else f"{it} + 1"
            return node.value.id if ast.unparse(node.slice) == want else None

        owned = {}      # loop variable -> pointer array

        def scan(statements, inherited):
            for statement in statements:
                for node in ([statement] if isinstance(statement, ast.For)
                             else []):
                    pointer = None
                    if _is_range_loop(node) and len(node.iter.args) == 2:
                        low, high = node.iter.args
                        upper = pointer_of(high, 1)
                        lower = pointer_of(low, 0)
                        if upper is not None and lower == upper:
                            pointer = upper
                        elif (upper is not None and inherited == upper
                              and isinstance(low, (ast.Name, ast.BinOp))
                              and _names_in(low) & set(owned)):
                            # range(own position + c, P[i + 1]): still inside
                            pointer = upper
                    if pointer is not None and isinstance(node.target, ast.Name):
                        owned[node.target.id] = pointer
                    scan(node.body, pointer or inherited)
                for field in ("body", "orelse"):
                    if isinstance(statement, (ast.If, ast.While)):
                        scan(getattr(statement, field, []), inherited)

        scan(body, None)
        candidates = {}
        for statement in body:
            for node in ast.walk(statement):
                targets = []
                if isinstance(node, ast.Assign):
                    targets = node.targets
                elif isinstance(node, ast.AugAssign):
                    targets = [node.target]
                for target in targets:
                    if (isinstance(target, ast.Subscript)
                            and isinstance(target.value, ast.Name)
                            and isinstance(target.slice, ast.Name)
                            and target.slice.id in owned
                            and target.value.id not in reduced
                            and kinds.arrays.get(target.value.id) == FLOAT):
                        candidates.setdefault(
                            target.value.id, set()).add(owned[target.slice.id])
        if len(candidates) != 1:
            return None
        (array, pointers), = candidates.items()
        if len(pointers) != 1:
            return None
        groups = max(1, self.threads_per_block // self.task_lanes)
        # entries per task: 32 where a wavefront holds several tasks; with a
        # wavefront per task the rows of real factors (hundreds of entries)
        # fit as well -- 8 KB per wavefront, 64 KB per CU at eight resident
        capacity = min(1024 if self.task_lanes == 64 else 32, 4096 // groups)
        if self.segment_capacity is not None:
            capacity = int(self.segment_capacity)
        if capacity < 8:
            return None
        return {"array": array, "pointer": next(iter(pointers)),
                "capacity": capacity}

    def _segment_lines(self):
        """(prologue, epilogue) of a task that stages its own segment."""
        plan = self._segment
        array, pointer = plan["array"], plan["pointer"]
        it = self.loop_iterator
        coherent = array in self._emitter.coherent_arrays
        load = (f"lcd_ld(&{array}[_lcd_seg_base + _q])" if coherent
                else f"{array}[_lcd_seg_base + _q]")
        store = (f"lcd_st(&{array}[_lcd_seg_base + _q], _lcd_seg[_q]);"
                 if coherent else f"{array}[_lcd_seg_base + _q] = _lcd_seg[_q];")
        def bound(offset):
            # the copy in task order when the node loads use one
            for name, source, delta in self._queue_node_loads:
                if (source, delta) == (pointer, offset):
                    return f"{name}[_task]"
            return f"{pointer}[{it} + {offset}]" if offset else f"{pointer}[{it}]"

        prologue = [
            f"_lcd_seg_base = {bound(0)};",
            f"_lcd_seg_limit = {bound(1)} - _lcd_seg_base;",
            *(["_lcd_seg_own = _lcd_seg_limit;"] if self._published else []),
            "if (_lcd_seg_limit > LCD_SEG_CAP) _lcd_seg_limit = 0;",
            "for (int _q = _lane; _q < _lcd_seg_limit; _q += LCD_TASK_LANES) "
            f"_lcd_seg[_q] = {load};",
            self.group_sync,
        ]
        epilogue = [
            self.group_sync,
            "for (int _q = _lane; _q < _lcd_seg_limit; _q += LCD_TASK_LANES) "
            + store,
        ]
        if self._published:
            # the messages first (consumers wait for them), then the array
            # itself; a segment too long for LDS was updated in place and is
            # read back
            epilogue = [
                self.group_sync,
                "for (int _q = _lane; _q < _lcd_seg_limit; _q += LCD_TASK_LANES) "
                "lcd_st(&_lcd_pub[_lcd_seg_base + _q], _lcd_seg[_q]);",
                "if (_lcd_seg_limit == 0) for (int _q = _lane; _q < _lcd_seg_own; "
                "_q += LCD_TASK_LANES) lcd_st(&_lcd_pub[_lcd_seg_base + _q], "
                f"lcd_ld(&{array}[_lcd_seg_base + _q]));",
                "for (int _q = _lane; _q < _lcd_seg_limit; _q += LCD_TASK_LANES) "
                f"{array}[_lcd_seg_base + _q] = _lcd_seg[_q];",
            ]
        return prologue, epilogue

    def _forward_stores(self, statements, mapped_loop):
        """``X[e] = value`` directly followed by ``name = X[e]``: every lane
        keeps ``value`` in a register instead of reading the element back
        through memory (a store -> fence -> load round trip on the task's
        critical path; ILU0's ``A_data[k_ptr] /= diag; l_ik = A_data[k_ptr]``).
        """
        lowerer = self
        counter = [0]

        def rewrite(block):
            out = []
            index = 0
            while index < len(block):
                first = block[index]
                second = block[index + 1] if index + 1 < len(block) else None
                if (isinstance(first, ast.Assign) and len(first.targets) == 1
                        and isinstance(first.targets[0], ast.Subscript)
                        and isinstance(first.targets[0].value, ast.Name)
                        and isinstance(second, ast.Assign)
                        and len(second.targets) == 1
                        and isinstance(second.targets[0], ast.Name)
                        and isinstance(second.value, ast.Subscript)
                        and ast.unparse(second.value)
                        == ast.unparse(first.targets[0])
                        and second.targets[0].id
                        not in _names_in(first.targets[0].slice)):
                    name = f"_lcd_fw_{counter[0]}"
                    counter[0] += 1
                    array = first.targets[0].value.id
                    lowerer._kinds.locals[name] = lowerer._kinds.arrays.get(
                        array, FLOAT)
                    lowerer._own_registers.append(name)
                    keep = ast.Assign(
                        targets=[ast.Name(id=name, ctx=ast.Store())],
                        value=first.value)
                    store = ast.Assign(
                        targets=first.targets,
                        value=ast.Name(id=name, ctx=ast.Load()))
                    reuse = ast.Assign(
                        targets=second.targets,
                        value=ast.Name(id=name, ctx=ast.Load()))
                    for new, old in ((keep, first), (store, first),
                                     (reuse, second)):
                        ast.copy_location(new, old)
                    out += [keep, store, reuse]
                    index += 2
                    continue
                if first is not mapped_loop:
                    for field in ("body", "orelse"):
                        inner = getattr(first, field, None)
                        if isinstance(inner, list) and inner and isinstance(
                                inner[0], ast.stmt):
                            setattr(first, field, rewrite(inner))
                out.append(first)
                index += 1
            return out

        result = rewrite(list(statements))
        ast.fix_missing_locations(ast.Module(body=result, type_ignores=[]))
        return result

    def _guard_stores(self, statements, mapped_loop):
        """Outside the mapped loop, array stores are issued by lane 0 of the
        group and followed by a group-scope fence."""
        lowerer = self

        class Guard(ast.NodeTransformer):
            def visit_For(self, node):
                if node is mapped_loop:
                    return node
                return self.generic_visit(node)

            def _guarded(self, node):
                marker = ast.If(
                    test=ast.Name(id="_LCD_LANE0", ctx=ast.Load()),
                    body=[node], orelse=[])
                marker._lcd_store_guard = True
                return ast.copy_location(marker, node)

            def visit_Assign(self, node):
                if any(isinstance(t, ast.Subscript) for t in node.targets):
                    return self._guarded(node)
                return node

            def visit_AugAssign(self, node):
                if isinstance(node.target, ast.Subscript):
                    location = (node.lineno, node.col_offset)
                    if location in lowerer.reductions:
                        return self._guarded(node)
                    return self._guarded(node)
                return node

        wrapper = ast.Module(body=statements, type_ignores=[])
        return Guard().visit(wrapper).body

    def _promote_own_elements(self, body, mapped, hooks, arguments):
        """Keep ``X[E]`` in a register for the whole task when ``E`` depends
        only on the block iterator and loop-invariant inputs and the task
        stores it at its top level (``x[i]`` of the triangular solves).

        Every lane of the group computes the value (uniform code, identical
        loads), the distributed loop reads the register instead of memory,
        and lane 0 stores it once at the end of the task, before successors
        are released.  This removes the store -> fence -> reload round trips
        from the task's dependency chain.  Other elements of ``X`` may only be
        touched inside the distributed loop (reads, atomic updates, or stores
        at loop-variant positions): a task's own element is never one of
        those, because the DAG has no self edges.
        """
        written = self._written_arrays(body)
        invariant_names = {self.loop_iterator} | {
            name for name in arguments if name not in written}
        invariant_names |= set(self._lifted_parameters)
        top_level = [s for s in body if s is not mapped]

        def own(node):
            return (isinstance(node, ast.Subscript)
                    and isinstance(node.value, ast.Name)
                    and node.value.id in written
                    and _names_in(node.slice) <= invariant_names
                    and not (_names_in(node.slice) & written))

        candidates = {}
        for statement in top_level:
            target = None
            if isinstance(statement, ast.Assign) and len(statement.targets) == 1:
                target = statement.targets[0]
            elif isinstance(statement, ast.AugAssign):
                target = statement.target
            if target is not None and own(target):
                if (isinstance(statement, ast.AugAssign)
                        and (statement.lineno, statement.col_offset)
                        in self.reductions):
                    continue
                candidates.setdefault(ast.dump(target.value) + "|"
                                      + ast.unparse(target.slice), target)
        for _, target, _ in (hooks.partials if hooks else []):
            if own(target):
                candidates.setdefault(ast.dump(target.value) + "|"
                                      + ast.unparse(target.slice), target)
        promoted = {}
        for key, target in candidates.items():
            array = target.value.id
            index_text = ast.unparse(target.slice)
            safe = True
            for statement in top_level:
                for node in ast.walk(statement):
                    if (isinstance(node, ast.Subscript)
                            and isinstance(node.value, ast.Name)
                            and node.value.id == array
                            and ast.unparse(node.slice) != index_text):
                        safe = False
            if any(other != key and other.split("|")[0] == key.split("|")[0]
                   for other in candidates):
                safe = False
            if safe:
                promoted[key] = (array, index_text,
                                 f"_lcd_own_{len(promoted)}", target)
        if not promoted:
            return body, [], []

        by_text = {(array, index_text): name
                   for array, index_text, name, _ in promoted.values()}
        first_access = {}   # name -> "read" | "write"

        class Replace(ast.NodeTransformer):
            def visit_Subscript(self, node):
                if isinstance(node.value, ast.Name):
                    name = by_text.get((node.value.id, ast.unparse(node.slice)))
                    if name is not None:
                        return ast.copy_location(
                            ast.Name(id=name, ctx=node.ctx), node)
                return self.generic_visit(node)

        def note(statement):
            reads, writes = set(), set()
            for node in ast.walk(statement):
                if isinstance(node, ast.Subscript) and isinstance(
                        node.value, ast.Name):
                    name = by_text.get((node.value.id, ast.unparse(node.slice)))
                    if name is None:
                        continue
                    if isinstance(node.ctx, ast.Store) and not isinstance(
                            statement, ast.AugAssign):
                        writes.add(name)
                    else:
                        reads.add(name)
            if isinstance(statement, ast.Assign):
                value_reads = set()
                for node in ast.walk(statement.value):
                    if isinstance(node, ast.Subscript) and isinstance(
                            node.value, ast.Name):
                        name = by_text.get(
                            (node.value.id, ast.unparse(node.slice)))
                        if name is not None:
                            value_reads.add(name)
                reads = value_reads | (reads - writes)
            for name in reads:
                first_access.setdefault(name, "read")
            for name in writes:
                first_access.setdefault(name, "write")

        for statement in body:
            note(statement)
        for _, target, _ in (hooks.partials if hooks else []):
            name = by_text.get((target.value.id, ast.unparse(target.slice))
                               ) if isinstance(target, ast.Subscript) else None
            if name is not None:
                first_access.setdefault(name, "read")
        replacer = Replace()
        new_body = []
        for statement in body:
            if statement is mapped:
                mapped.body = [replacer.visit(s) for s in mapped.body]
                new_body.append(mapped)
            else:
                new_body.append(replacer.visit(statement))
        if hooks:
            hooks.partials = [
                (partial, replacer.visit(deepcopy(target)), op)
                for partial, target, op in hooks.partials]
        if self.direct_dependence is not None:
            pass   # endpoints never name an own element
        prologue, epilogue = [], []
        emitter = self._emitter
        for array, index_text, name, target in promoted.values():
            self._own_map[f"{array}[{index_text}]"] = (
                name, first_access.get(name, "read"))
            self._kinds.locals[name] = self._kinds.arrays.get(array, FLOAT)
            self._own_registers.append(name)
            load_node = ast.Subscript(
                value=ast.Name(id=array, ctx=ast.Load()),
                slice=deepcopy(target.slice), ctx=ast.Load())
            if first_access.get(name, "read") == "read":
                if (array in self._own_zero_arrays or (
                        self._value_pull is not None
                        and self._value_pull["array"] == array)):
                    # still its initial zero: no other task writes it, and
                    # the executor does not clear the array
                    prologue.append(f"{name} = 0.0;")
                else:
                    prologue.append(f"{name} = {emitter.expr(load_node)};")
            epilogue.append("if (_lane == 0) " + emitter.store(load_node, name))
        ast.fix_missing_locations(ast.Module(body=new_body, type_ignores=[]))
        return new_body, prologue, epilogue

    def _hoist_node_loads(self, body, mapped, arguments):
        """Issue a task's read-only loads before it waits for its producers.

        Loads ``R[e]`` of arrays the kernel never writes whose index depends
        only on the block iterator and loop-invariant inputs (``Ap[i]``,
        ``b[i]``, ``Ax[Ap[i]]``) are moved into registers right after the
        task is fetched (the reference prefetches node loads before its spin,
        compiler/cuda_lowering.py:1991-2029).  For a top-level distributed
        loop the loads of each lane's *first* iteration (``Ai[j]``,
        ``Ax[j]``) are issued there as well, so that after the wait only the
        data other tasks produce is still to be fetched.
        """
        kinds = self._kinds
        written = self._all_written      # as written by the original loop
        readonly = {name for name in kinds.arrays if name not in written}
        invariant = {self.loop_iterator} | {
            name for name in arguments if name not in kinds.arrays}
        invariant |= set(self._lifted_parameters)
        temps = {}          # unparse text -> (temp name, load node)
        order = []
        lowerer = self

        def hoistable(node, extra=()):
            if not (isinstance(node, ast.Subscript)
                    and isinstance(node.value, ast.Name)
                    and node.value.id in readonly
                    and isinstance(node.ctx, ast.Load)):
                return False
            allowed = invariant | set(extra) | {
                name for name, _ in temps.values()
                if name.startswith("_nl_") or extra}
            for sub in ast.walk(node.slice):
                if isinstance(sub, ast.Name) and sub.id not in allowed and (
                        sub.id not in readonly):
                    return False
                if isinstance(sub, ast.Call):
                    return False
            return True

        class Hoist(ast.NodeTransformer):
            def __init__(self, prefix, extra=()):
                self.prefix = prefix
                self.extra = extra

            def visit_Subscript(self, node):
                node = self.generic_visit(node)   # innermost first
                if not hoistable(node, self.extra):
                    return node
                text = ast.unparse(node)
                if text not in temps:
                    name = f"{self.prefix}{len(temps)}"
                    temps[text] = (name, deepcopy(node))
                    order.append(text)
                    kinds.locals[name] = kinds.arrays.get(node.value.id, FLOAT)
                return ast.copy_location(
                    ast.Name(id=temps[text][0], ctx=ast.Load()), node)

        def visit_unconditional(statement, transformer):
            if isinstance(statement, ast.Assign):
                statement.value = transformer.visit(statement.value)
                for target in statement.targets:
                    if isinstance(target, ast.Subscript):
                        target.slice = transformer.visit(target.slice)
            elif isinstance(statement, ast.AugAssign):
                statement.value = transformer.visit(statement.value)
                if isinstance(statement.target, ast.Subscript):
                    statement.target.slice = transformer.visit(
                        statement.target.slice)
            return statement

        node_hoist = Hoist("_nl_")
        for statement in body:
            if statement is mapped:
                mapped.iter.args = [node_hoist.visit(a) for a in mapped.iter.args]
                for inner in mapped.body:
                    visit_unconditional(inner, node_hoist)
            else:
                visit_unconditional(statement, node_hoist)
        node_count = len(order)
        first_iteration = []
        if (mapped is not None and mapped in body
                and self.thread_unroll_factor == 1 and len(mapped.iter.args) == 2):
            lane_hoist = Hoist("_pf_", extra=(mapped.target.id,))
            for inner in mapped.body:
                visit_unconditional(inner, lane_hoist)
            if self._mailbox is not None:
                # the message slot of this lane's position loads with the
                # first iteration's operands, ahead of the wait
                self._mailbox["slot"] = lane_hoist.visit(
                    self._mailbox_slot_load())
            first_iteration = order[node_count:]
            if self.direct_dependence is not None and first_iteration:
                dependence = self.direct_dependence
                self._hook_endpoint = lane_hoist.visit(deepcopy(dependence.endpoint))
                self._hook_guard = (lane_hoist.visit(deepcopy(dependence.guard))
                                    if dependence.guard is not None else None)
                # the hook may not create new prefetches
                first_iteration = order[node_count:]
        elif self.direct_dependence is not None:
            pass
        emitter = self._emitter
        prefetch = []
        for text in order[:node_count]:
            name, node = temps[text]
            queued = self._queue_node_load(node)
            if queued is not None:
                # addressed by the queue position: issued with the task id
                self._queue_load_lines.append(f"{name} = {queued}[_task];")
            else:
                prefetch.append(f"{name} = {emitter.expr(node)};")
        self._own_registers.extend(temps[text][0] for text in order)
        reload_lines = []
        if first_iteration:
            lower, upper, _ = emitter.range_parts(mapped)
            it = mapped.target.id
            loads = " ".join(
                f"{temps[text][0]} = {emitter.expr(temps[text][1])};"
                for text in first_iteration)
            prefetch.append(f"{it} = ({lower}) + _lane;")
            prefetch.append(f"if ({it} < {upper}) {{ {loads} }}")
            reload_lines = [f"if ({it} != ({lower}) + _lane) {{ {loads} }}"]
        self._first_iteration_reload = reload_lines
        ast.fix_missing_locations(ast.Module(body=body, type_ignores=[]))
        return body, prefetch

    def _queue_node_load(self, node):
        """``P[i + c]`` of a structure array ``P`` (one whose contents are
        part of the inspection fingerprint): read it from a copy in task
        order, ``_lcd_qn_k[_task]``, which the runtime gathers once per
        structure -- one load less on the chain in front of every task."""
        # persistent executors whose hand-offs are the values themselves
        # only: measured 1-2 % there; level launches lose 4 % and the flagged
        # pull 1 % (ILU0, 9-point grid) because rows of consecutive levels
        # are neighbours, so `Ap[i]` is warm in L2 from the level before
        # while a queue-ordered copy is cold at every level
        value_flags = self._value_pull is not None or (
            self._mailbox is not None and self._mailbox["gather"] is not None)
        if (not self.queue_node_loads_enabled or self.chain_tasks
                or not self.warp_mapped or self.execution_mode != "sync_free"
                or not value_flags):
            return None
        array = node.value.id
        properties = (self.function_props or {}).get(array, ())
        if "monotonically_increasing" not in properties:
            return None
        base, offset = _split_offset(node.slice)
        if not (isinstance(base, ast.Name) and base.id == self.loop_iterator):
            return None
        for name, source, delta in self._queue_node_loads:
            if (source, delta) == (array, offset):
                return name
        name = f"_lcd_qn_{len(self._queue_node_loads)}"
        self._queue_node_loads.append((name, array, offset))
        self._kinds.arrays[name] = INT
        return name

    def _task_body(self, body, emitter, local_names, target_loop, arguments):
        """C++ lines of one task (indent level 0), `i` already bound."""
        gather = self._mailbox["gather"] if self._mailbox is not None else None
        if gather is not None:
            # the consumers form the products themselves: the producer's
            # distributed loop is gone
            site = self._mailbox["sites"][0]
            body = [s for s in body if s is not self._mailbox["mapped"]]
            emitter.lowered_ids.add(
                self.reductions[(site.lineno, site.col_offset)][0])
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
            if own is None or own[1] != "read":
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
            lines.extend(self._emit_guarded(statement, emitter, 0, hooks))
        lines.extend(epilogue)
        return lines

    def _emit_guarded(self, node, emitter, indent, hooks):
        pad = "    " * indent
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

    def _sequential_pull_lines(self, node, emitter, hooks, lower, upper):
        """The task's loop over its producers, resumable: every iteration
        first checks that its producer has published ``done`` and otherwise
        leaves the loop with the position kept; the lines between the two
        markers are re-entered by the executor's poll loop.  The task works
        on the producers that are finished while it waits for the others."""
        plan = self._sequential_pull
        plan["emitted"] = True
        name = node.target.id
        # the wait goes after the statements that leave the loop at the
        # task's own entry (`if k >= i: break`)
        split = 0
        for position, statement in enumerate(node.body):
            if (isinstance(statement, ast.If) and len(statement.body) == 1
                    and isinstance(statement.body[0], ast.Break)
                    and not statement.orelse):
                split = position + 1
                break
        # ... and after the plain assignments that follow and read nothing
        # another task writes (`diag_ptr = lookup[k]`): structure loads that
        # would otherwise sit between the wait and the first use of row k
        # From the first search on (`diag_ptr = find(row k, k)`) they run
        # once per iteration instead of once per poll.
        searches = None
        while split < len(node.body):
            statement = node.body[split]
            if not (isinstance(statement, ast.Assign)
                    and all(isinstance(t, ast.Name) for t in statement.targets)):
                break
            if any(isinstance(sub, ast.Subscript)
                   and isinstance(sub.value, ast.Name)
                   and sub.value.id in self._all_written
                   for sub in ast.walk(statement)):
                break
            calls = [sub for sub in ast.walk(statement)
                     if isinstance(sub, ast.Call)]
            if any(not (isinstance(call.func, ast.Name)
                        and call.func.id == "_lcd_sorted_find")
                   for call in calls):
                break
            if calls and searches is None:
                searches = split
            split += 1
        once = [] if searches is None else node.body[searches:split]
        every_poll = split if searches is None else searches
        early, fetched = self._locate_ahead_of_wait(node.body[split:], hooks)
        early = list(once) + early
        if self._published is not None and self.look_ahead:
            lines = self._pipelined_pull_lines(
                node, emitter, hooks, lower, every_poll, split, early, fetched)
            if lines is not None:
                return lines
        endpoint = emitter.expr(plan["endpoint"])
        waiting = f"lcd_load_relaxed(&done[{endpoint}]) == 0"
        blocked = (f"!lcd_group_none({waiting})" if self.task_lanes > 1
                   else waiting)
        if early:
            # once per iteration of the producer loop, not once per poll
            self._own_registers.append("_sp_at")
            self._kinds.locals["_sp_at"] = INT
            early = [ast.fix_missing_locations(ast.If(
                test=ast.Compare(left=ast.Name(id="_sp_at", ctx=ast.Load()),
                                 ops=[ast.NotEq()],
                                 comparators=[ast.Name(id=name, ctx=ast.Load())]),
                body=[ast.Assign(
                    targets=[ast.Name(id="_sp_at", ctx=ast.Store())],
                    value=ast.Name(id=name, ctx=ast.Load())), *early],
                orelse=[]))]
        lines = [f"{name} = {lower};",
                 *(["_sp_at = -1;"] if early else []), VALUE_WAIT_BEGIN,
                 "_lcd_blocked = false;",
                 f"for (; {name} < {upper}; ++{name}) {{"]
        for child in node.body[:every_poll]:
            lines += self._emit_guarded(child, emitter, 1, hooks)
        for child in early:
            lines += self._emit_guarded(child, emitter, 1, hooks)
        if self._published is None:
            lines += [f"    if ({blocked}) {{ _lcd_blocked = true; break; }}",
                      "    lcd_acquire_fence();"]
        for child in fetched:
            lines += self._emit_guarded(child, emitter, 1, hooks)
        for child in node.body[split:]:
            lines += self._emit_guarded(child, emitter, 1, hooks)
        lines += ["}", VALUE_WAIT_END]
        return lines

    def _pipelined_pull_lines(self, node, emitter, hooks, lower, every_poll,
                              split, structure, fetched):
        """The producer loop with published values, one iteration ahead in
        its structure work.  An iteration issues the first loads of its
        producer's values, then locates what the *next* iteration will read
        (the next producer's row is searched while this one's values are on
        their way or not even stored yet), then waits for its values and
        works.  What is left between the arrival of a producer's values and
        the publication of the task's own is arithmetic."""
        name = node.target.id
        upper = node.iter.args[1]
        leading = list(node.body[:every_poll])
        leave = next((position for position, statement in enumerate(leading)
                      if isinstance(statement, ast.If)
                      and len(statement.body) == 1
                      and isinstance(statement.body[0], ast.Break)), None)
        before = leading if leave is None else leading[:leave]
        after = [] if leave is None else leading[leave + 1:]
        if not all(isinstance(statement, ast.Assign) and all(
                isinstance(target, ast.Name) for target in statement.targets)
                   for statement in before + after):
            return None
        # everything an iteration sets up before it reads its producer is
        # located one iteration ahead, `diag_ptr = table[k]` included
        structure = after + list(structure)
        located = before + structure
        names = []
        for statement in located:
            for sub in ast.walk(statement):
                if (isinstance(sub, ast.Name) and isinstance(sub.ctx, ast.Store)
                        and sub.id not in names):
                    names.append(sub.id)
        kinds = self._kinds
        for local in names:
            kinds.locals[f"_nx_{local}"] = kinds.locals.get(local, INT)
            self._own_registers.append(f"_nx_{local}")

        def ahead(offset):
            position = (ast.Name(id=name, ctx=ast.Load()) if offset == 0 else
                        ast.BinOp(left=ast.Name(id=name, ctx=ast.Load()),
                                  op=ast.Add(), right=ast.Constant(value=offset)))

            class Shift(ast.NodeTransformer):
                def visit_Name(self, sub):
                    if sub.id in names:
                        return ast.copy_location(
                            ast.Name(id=f"_nx_{sub.id}", ctx=sub.ctx), sub)
                    if sub.id == name:
                        return ast.copy_location(deepcopy(position), sub)
                    return sub

            shifted = [Shift().visit(deepcopy(statement))
                       for statement in before]
            body = [Shift().visit(deepcopy(statement)) for statement in structure]
            if leave is not None:
                body = [ast.If(test=ast.UnaryOp(
                    op=ast.Not(), operand=Shift().visit(
                        deepcopy(leading[leave].test))), body=body, orelse=[])]
            return ast.fix_missing_locations(ast.If(
                test=ast.Compare(left=deepcopy(position), ops=[ast.Lt()],
                                 comparators=[deepcopy(upper)]),
                body=shifted + body, orelse=[]))

        rest = list(node.body[split:])
        leading_loads = self._split_leading_loads(rest)
        first_loads = list(fetched) + leading_loads
        take_over = [ast.fix_missing_locations(ast.Assign(
            targets=[ast.Name(id=local, ctx=ast.Store())],
            value=ast.Name(id=f"_nx_{local}", ctx=ast.Load())))
            for local in names]
        lines = [f"{name} = {lower};"]
        lines += self._emit_guarded(ahead(0), emitter, 0, hooks)
        lines += [VALUE_WAIT_BEGIN, "_lcd_blocked = false;",
                  f"for (; {name} < {emitter.expr(upper)}; ++{name}) {{"]
        for child in take_over + ([] if leave is None else [leading[leave]]):
            lines += self._emit_guarded(child, emitter, 1, hooks)
        # the next producer's row is searched while this one's values are on
        # their way.  (Sending the next one's first loads too, once these
        # values are here, was slower: 8.2 against 7.2 ms on the 9-point
        # grid -- the compiler waits for them where the guarded loads meet.)
        for child in first_loads + [ahead(1)] + rest:
            lines += self._emit_guarded(child, emitter, 1, hooks)
        lines += ["}", VALUE_WAIT_END]
        return lines

    def _split_leading_loads(self, rest):
        """Leading statements of the form ``[if structure:] x = X[p]`` (the
        producer's diagonal): the first attempt of the load is issued with
        the other first loads and the statement waits for the value.
        Returns the issuing statements; ``rest`` is rewritten in place."""
        issued = []

        def structural(expression):
            return not any(
                isinstance(sub, ast.Call) or (
                    isinstance(sub, ast.Subscript)
                    and isinstance(sub.value, ast.Name)
                    and sub.value.id in self._all_written)
                for sub in ast.walk(expression))

        def split_assign(assign):
            if not (isinstance(assign, ast.Assign) and len(assign.targets) == 1
                    and isinstance(assign.targets[0], ast.Name)
                    and isinstance(assign.value, ast.Subscript)
                    and isinstance(assign.value.value, ast.Name)
                    and assign.value.value.id == self._published["array"]
                    and structural(assign.value.slice)):
                return None
            register = f"_sp_ld_h{len(issued)}"
            self._kinds.locals[register] = FLOAT
            self._own_registers.append(register)
            load = ast.Assign(
                targets=[ast.Name(id=register, ctx=ast.Store())],
                value=ast.Call(func=ast.Name(id="_lcd_raw", ctx=ast.Load()),
                               args=[deepcopy(assign.value)], keywords=[]))
            assign.value = ast.Call(
                func=ast.Name(id="_lcd_settle", ctx=ast.Load()),
                args=[assign.value, ast.Name(id=register, ctx=ast.Load())],
                keywords=[])
            return load

        for statement in rest:
            if (isinstance(statement, ast.If) and not statement.orelse
                    and structural(statement.test)
                    and len(statement.body) == 1):
                load = split_assign(statement.body[0])
                if load is None:
                    break
                issued.append(ast.If(test=deepcopy(statement.test),
                                     body=[load], orelse=[]))
            else:
                load = split_assign(statement)
                if load is None:
                    break
                issued.append(load)
        for statement in issued + rest:
            ast.fix_missing_locations(statement)
        return issued

    def _locate_ahead_of_wait(self, statements, hooks):
        """The thread-mapped loop nested in a resumable producer loop starts
        with structure work (`j = A_indices[j_ptr]; kj_ptr = find(...)`)
        that reads nothing another task writes.  For each lane's first
        iteration it is done ahead of the wait for the producer (into
        ``_sp_*`` registers the loop then picks up), which takes the search
        of the pivot row off the chain between two levels.  Returns the
        statements to run before the wait; the loop is rewritten in place."""
        if hooks is None or self.thread_unroll_factor != 1:
            return [], []
        mapped = None
        for statement in statements:
            for sub in ast.walk(statement):
                if isinstance(sub, ast.For) and hooks.is_mapped(sub):
                    mapped = sub
        if mapped is None or len(mapped.iter.args) != 2 or not isinstance(
                mapped.target, ast.Name):
            return [], []
        iterator = mapped.target.id
        structural = []
        for statement in mapped.body:
            if not (isinstance(statement, ast.Assign)
                    and len(statement.targets) == 1
                    and isinstance(statement.targets[0], ast.Name)):
                break
            reads_written = any(
                isinstance(sub, ast.Subscript) and isinstance(sub.value, ast.Name)
                and sub.value.id in self._all_written
                for sub in ast.walk(statement))
            calls = [sub for sub in ast.walk(statement)
                     if isinstance(sub, ast.Call)]
            if reads_written or any(
                    not (isinstance(call.func, ast.Name)
                         and call.func.id == "_lcd_sorted_find")
                    for call in calls):
                break
            structural.append(statement)
        if not structural:
            return [], []
        names = {statement.targets[0].id for statement in structural}
        renamed = {name: f"_sp_{name}" for name in names}
        renamed[iterator] = "_sp_first"

        class Rename(ast.NodeTransformer):
            def visit_Name(self, node):
                if node.id in renamed:
                    return ast.copy_location(
                        ast.Name(id=renamed[node.id], ctx=node.ctx), node)
                return node

        kinds = self._kinds
        for name in names:
            kinds.locals[renamed[name]] = kinds.locals.get(name, INT)
        kinds.locals["_sp_first"] = INT
        self._own_registers.extend(["_sp_first", *sorted(
            renamed[name] for name in names)])
        lower, upper = mapped.iter.args
        first = ast.Assign(
            targets=[ast.Name(id="_sp_first", ctx=ast.Store())],
            value=ast.BinOp(left=deepcopy(lower), op=ast.Add(),
                            right=ast.Name(id="_lane", ctx=ast.Load())))
        ahead = ast.If(
            test=ast.Compare(left=ast.Name(id="_sp_first", ctx=ast.Load()),
                             ops=[ast.Lt()], comparators=[deepcopy(upper)]),
            body=[Rename().visit(deepcopy(statement))
                  for statement in structural],
            orelse=[])
        pick_up = ast.If(
            test=ast.Compare(left=ast.Name(id=iterator, ctx=ast.Load()),
                             ops=[ast.Eq()],
                             comparators=[ast.Name(id="_sp_first",
                                                   ctx=ast.Load())]),
            body=[ast.Assign(
                targets=[ast.Name(id=statement.targets[0].id, ctx=ast.Store())],
                value=ast.Name(id=renamed[statement.targets[0].id],
                               ctx=ast.Load())) for statement in structural],
            orelse=list(structural))
        rest = mapped.body[len(structural):]
        fetched = self._fetch_behind_wait(rest, iterator, names, renamed, upper)
        mapped.body = [pick_up] + rest
        early = [first, ahead]
        for statement in early + fetched + [pick_up]:
            ast.fix_missing_locations(statement)
        return early, fetched

    def _fetch_behind_wait(self, rest, iterator, names, renamed, upper):
        """After the structure work the nested loop reads the producer's
        values at the positions just found (`if kj_ptr >= 0: u = A[kj_ptr]`).
        For each lane's first iteration those loads are issued right behind
        the wait, together with the first load the task makes of the
        producer (its diagonal), instead of one dependent round trip later.
        Valid because a pull rule means the task writes only its own element
        or segment: nothing it does in between changes what it reads here."""
        if not (rest and isinstance(rest[0], ast.If) and not rest[0].orelse):
            return []
        guard = rest[0]
        known = set(names)
        for sub in ast.walk(guard.test):
            if isinstance(sub, (ast.Subscript, ast.Call)) or (
                    isinstance(sub, ast.Name) and sub.id == iterator):
                return []
        loads = {}
        published = self._published is not None

        def eligible(node):
            if not (isinstance(node, ast.Subscript)
                    and isinstance(node.ctx, ast.Load)
                    and isinstance(node.value, ast.Name)
                    and node.value.id in self._all_written):
                return False
            used = {n.id for n in ast.walk(node.slice)
                    if isinstance(n, ast.Name)}
            if iterator in used or not (used & known):
                return False
            return not any(isinstance(n, (ast.Subscript, ast.Call))
                           for n in ast.walk(node.slice))

        class Hoist(ast.NodeTransformer):
            def visit_Subscript(self, node):
                if not eligible(node):
                    return self.generic_visit(node)
                text = ast.unparse(node)
                if text not in loads:
                    loads[text] = (f"_sp_ld_{len(loads)}", deepcopy(node))
                held = ast.Name(id=loads[text][0], ctx=ast.Load())
                if published:
                    # the first attempt may have met the empty marker
                    held = ast.Call(
                        func=ast.Name(id="_lcd_settle", ctx=ast.Load()),
                        args=[deepcopy(node), held], keywords=[])
                return ast.copy_location(ast.IfExp(
                    test=ast.Compare(
                        left=ast.Name(id=iterator, ctx=ast.Load()),
                        ops=[ast.Eq()],
                        comparators=[ast.Name(id="_sp_first", ctx=ast.Load())]),
                    body=held, orelse=node), node)

        # only loads the guarded block makes unconditionally
        guard.body = [
            Hoist().visit(statement) if isinstance(
                statement, (ast.Assign, ast.AugAssign)) else statement
            for statement in guard.body]
        if not loads:
            return []

        class Rename(ast.NodeTransformer):
            def visit_Name(self, node):
                if node.id in renamed:
                    return ast.copy_location(
                        ast.Name(id=renamed[node.id], ctx=node.ctx), node)
                return node

        kinds = self._kinds
        body = []
        for name, node in loads.values():
            kinds.locals[name] = kinds.arrays.get(node.value.id, FLOAT)
            self._own_registers.append(name)
            value = Rename().visit(node)
            if published:
                value = ast.Call(func=ast.Name(id="_lcd_raw", ctx=ast.Load()),
                                 args=[value], keywords=[])
            body.append(ast.Assign(
                targets=[ast.Name(id=name, ctx=ast.Store())], value=value))
        test = ast.BoolOp(op=ast.And(), values=[
            ast.Compare(left=ast.Name(id="_sp_first", ctx=ast.Load()),
                        ops=[ast.Lt()], comparators=[deepcopy(upper)]),
            Rename().visit(deepcopy(guard.test))])
        return [ast.If(test=test, body=body, orelse=[])]

    # ---- text assembly
    def _c_type(self, name, kind, is_array):
        return f"LCD_T_{name}"

    def _module_text(self, array_arguments, scalar_arguments, reset_text,
                     kernel_text):
        defines = [
            "#ifndef LCD_INDEX_TYPE", "#define LCD_INDEX_TYPE int", "#endif",
            f"#define LCD_TPB {self.threads_per_block}",
            f"#define LCD_TASK_LANES {self.task_lanes}",
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
        if self._segment is not None:
            defines.append(f"#define LCD_SEG_CAP {self._segment['capacity']}")
        if self._tile is not None:
            defines.append(f"#define LCD_TILE_ROWS {self._tile['rows']}")
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
                            STATUS_ARGUMENT, "_lcd_mailbox", "_lcd_pub"}
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
                     + list(self._own_registers)):
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
        if self._tile is not None:
            lines += [
                f"    __shared__ LCD_T_{self._tile['array']} "
                "_lcd_tile[LCD_TILE_ROWS];",
                "    lcd_index_t _lcd_tile_row0 = 0, _lcd_tile_rows = 0;",
            ]
        if self._segment is not None:
            array = self._segment["array"]
            lines += [
                f"    __shared__ LCD_T_{array} _lcd_seg_store["
                "LCD_GROUPS_PER_BLOCK * LCD_SEG_CAP];",
                f"    LCD_T_{array}* const _lcd_seg = &_lcd_seg_store["
                "(threadIdx.x / LCD_TASK_LANES) * LCD_SEG_CAP];",
                "    lcd_index_t _lcd_seg_base = 0, _lcd_seg_limit = 0;",
                *(["    lcd_index_t _lcd_seg_own = 0;"] if self._published else []),
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
            if self.execution_mode != "sync_free":
                out += [pad + "    " + line for line in prefetch]
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
            return [f"{pad}{it} = task_nodes[_task];",
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
        if self.chain_tasks:
            raise HIPLoweringError(
                "band_width > 1 (chain tasks) needs the wavefront executor.")
        lines = ["    const int _task_count = (int)task_count;"]
        if self.block_task:
            lines += [
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
                "                if (++_spins > LCD_SPIN_LIMIT || ((_spins & 255) == 0 && "
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
            # tile is always running and depends on finished tiles only
            fetch = [
                "    for (int _tile = blockIdx.x; (long long)_tile * LCD_TILE_ROWS "
                "< _task_count; _tile += gridDim.x) {",
                "    _lcd_tile_row0 = _tile * LCD_TILE_ROWS;",
                "    _lcd_tile_rows = _task_count - _lcd_tile_row0 < LCD_TILE_ROWS "
                "? _task_count - _lcd_tile_row0 : LCD_TILE_ROWS;",
                "    for (int _s = threadIdx.x; _s < _lcd_tile_rows; _s += LCD_TPB) "
                "_lcd_tile[_s] = lcd_empty();",
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
        lines += [
            "    const int _tasks_per_wave = 64 / LCD_TASK_LANES;",
            *fetch,
            *([f"        {it} = 0;"] if records else
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
            "                    _pending = false;",
            "                } else {",
            "#if LCD_SPIN_SLEEP > 0",
            "                    __builtin_amdgcn_s_sleep(LCD_SPIN_SLEEP);",
            "#endif",
            # the watchdog looks up once in 1024 polls (a 32-bit counter, one
            # test per poll): kept out of the way of the hand-offs, it costs
            # 3 % on the 128^3 grid where the test per poll cost 8 %
            "                    if ((++_spins & 1023u) == 0u && (_spins > "
            "(unsigned)LCD_SPIN_LIMIT || "
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
        return lines

    def _gather_fetch_lines(self, indent, declare=False, records=False):
        """Position, source and read-only operands of the incoming edge this
        lane handles next (slot ``_mb_next + _lane``); with ``records`` the
        first chunk comes from the task's fixed-size record."""
        pad = "    " * indent
        gather = self._mailbox["gather"]
        emitter = self._emitter
        lines = []
        if declare:
            lines.append(f"{pad}lcd_index_t _g_pos = 0, _g_src = 0;")
            lines.append(f"{pad}double _mb_value = lcd_empty();")
            for name, _, kind in gather["operands"]:
                ctype = "lcd_index_t" if kind == INT else "double"
                lines.append(f"{pad}{ctype} {name} = 0;")
        staged = gather["staged"]
        loads = " ".join(
            f"{name} = {staged[name]}[_mb_next + _lane];" if name in staged
            else f"{name} = {emitter.expr(node)};"
            for name, node, _ in gather["operands"])
        head = "if (_pending && _mb_next + _lane < _mb_end)" if declare else (
            "if (_mb_next + _lane < _mb_end)")
        decode = ("_g_off = (unsigned)(_g_src - _lcd_tile_row0); "
                  "_g_in = _g_off < (unsigned)_lcd_tile_rows; "
                  if self._tile is not None else "")
        if declare and self._tile is not None:
            lines.append(f"{pad}unsigned _g_off = 0; bool _g_in = false;")
        if records:
            # one guarded block, so the loads leave back to back
            slot = "_task * LCD_TASK_LANES + _lane"   # < 2^31 entries
            lines.append(
                f"{pad}if (_pending) {{ {self.loop_iterator} = "
                "(lcd_index_t)task_nodes[_task]; "
                "_mb_next = _lcd_rec_in[2 * _task]; "
                "_mb_end = _lcd_rec_in[2 * _task + 1]; "
                f"_g_pos = _lcd_rec_pos[{slot}]; "
                f"_g_src = _lcd_rec_src[{slot}]; {decode}"
                + " ".join(self._queue_load_lines) + " }")
            lines.append(f"{pad}{head} {{ {loads} }}")
            if self.single_chunk:
                lines += [
                    f"{pad}const int _mb_have = (_mb_end - _mb_next) < "
                    "LCD_TASK_LANES ? (_mb_end - _mb_next) : LCD_TASK_LANES;",
                    f"{pad}bool _need = _pending && _lane < _mb_have;",
                    # more incoming edges than lanes: never ready (watchdog)
                    f"{pad}const bool _fits = (_mb_end - _mb_next) <= "
                    "LCD_TASK_LANES;"]
            return lines
        position = ("_g_pos = _lcd_in_pos[_mb_next + _lane]; "
                    if gather["needs_position"] else "")
        lines.append(
            f"{pad}{head} {{ {position}"
            f"_g_src = _lcd_in_src[_mb_next + _lane]; {decode}{loads} }}")
        return lines

    def _gather_ready_lines(self, indent):
        """Readiness for the gathered mailbox: lane ``l`` polls the final
        value of the producer of incoming edge ``next + l`` until it is there
        and keeps the product; once the lanes of a chunk all hold theirs, the
        products are added in (source, position) order -- the order of the
        sequential loop -- by broadcasting them lane by lane."""
        pad = "    " * indent
        own = self._mailbox["register"]
        gather = self._mailbox["gather"]
        array = self._mailbox["array"]
        value = self._emitter.expr(gather["value"])
        if gather["negate"]:
            value = f"(-({value}))"
        tiled = self._tile is not None
        # in a tile the source was decoded when it was fetched (LDS slot or
        # not), the poll keeps the raw value and the product with the
        # operands is formed once the chunk is complete: a poll of the LDS
        # copy then waits for no load from memory
        load = ("(_g_in ? __hip_atomic_load(&_lcd_tile[_g_off], "
                "__ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) : "
                f"{self.poll_load}(&{array}[_g_src]))" if tiled
                else f"{self.poll_load}(&{array}[_g_src])")
        missing = "(_lane < _mb_have && lcd_is_empty(_mb_value))"
        complete = (f"lcd_group_none({missing})" if self.task_lanes > 1
                    else f"!{missing}")
        unroll = ([f"{pad}#pragma unroll"] if self.task_lanes <= 8 else [])
        bound = "LCD_TASK_LANES" if self.task_lanes <= 8 else "_mb_have"
        if self.task_lanes == 4:
            # four lanes per task: the ordered sum is four quad broadcasts
            ordered = [
                f"{pad}        {{ const double _mb_in = lcd_quad_broadcast<{k}>(_mb_value); "
                f"if ({k} < _mb_have) {own} = {own} + _mb_in; }}"
                for k in range(4)]
        else:
            ordered = [
                *unroll,
                f"{pad}        for (int _mb_k = 0; _mb_k < {bound}; ++_mb_k) {{",
                f"{pad}            const double _mb_in = __shfl(_mb_value, _mb_k, LCD_TASK_LANES);",
                f"{pad}            if (_mb_k < _mb_have) {own} = {own} + _mb_in;",
                f"{pad}        }}"]
        if self.single_chunk and gather.get("records"):
            # one chunk per task: what each lane still waits for is a flag
            # set when the task is fetched and cleared by its poll
            memory_poll = (
                f"{{ const double _g_raw = {self.poll_load}(&{array}[_g_src]); "
                "if (!lcd_is_empty(_g_raw)) { _mb_value = _g_raw; "
                "_need = false; } }")
            return [
                f"{pad}bool _ready = false;",
                f"{pad}if (_need) {{",
                *([f"{pad}    if (_g_in) {{ const double _g_raw = "
                   "__hip_atomic_load(&_lcd_tile[_g_off], __ATOMIC_RELAXED, "
                   "__HIP_MEMORY_SCOPE_WORKGROUP); "
                   "if (!lcd_is_empty(_g_raw)) { _mb_value = _g_raw; "
                   "_need = false; } }",
                   f"{pad}    else if ((_spins & LCD_EXTERNAL_POLL_MASK) == 0) "
                   + memory_poll] if tiled else
                  [f"{pad}    {memory_poll}"]),
                f"{pad}}}",
                f"{pad}if (_fits && lcd_group_none(_need)) {{",
                f"{pad}    if (_lane < _mb_have) {{ const double _g_value = "
                f"_mb_value; _mb_value = {value}; }}",
                *[line[4:] for line in ordered],
                f"{pad}    _ready = true;",
                f"{pad}}}",
            ]
        return [
            f"{pad}bool _ready = _mb_next == _mb_end;",
            f"{pad}if (!_ready) {{",
            f"{pad}    const int _mb_have = (_mb_end - _mb_next) < LCD_TASK_LANES ? "
            "(_mb_end - _mb_next) : LCD_TASK_LANES;",
            f"{pad}    if (_lane < _mb_have && lcd_is_empty(_mb_value)) {{",
            # two branches with their own temporaries: a wavefront whose
            # sources all sit in the tile never waits on the memory counter
            *([f"{pad}        if (_g_in) {{ const double _g_raw = "
               "__hip_atomic_load(&_lcd_tile[_g_off], __ATOMIC_RELAXED, "
               "__HIP_MEMORY_SCOPE_WORKGROUP); "
               "if (!lcd_is_empty(_g_raw)) _mb_value = _g_raw; }",
               f"{pad}        else if ((_spins & LCD_EXTERNAL_POLL_MASK) == 0) "
               f"{{ const double _g_raw = {self.poll_load}(&{array}[_g_src]); "
               "if (!lcd_is_empty(_g_raw)) _mb_value = _g_raw; }"]
              if tiled else
              [f"{pad}        const double _g_value = {load};",
               f"{pad}        if (!lcd_is_empty(_g_value)) _mb_value = {value};"]),
            f"{pad}    }}",
            f"{pad}    if ({complete}) {{",
            *([f"{pad}        if (_lane < _mb_have) {{ const double _g_value = "
               f"_mb_value; _mb_value = {value}; }}"] if tiled else []),
            *ordered,
            f"{pad}        _mb_next += _mb_have;",
            f"{pad}        _mb_value = lcd_empty();",
            # no task of this DAG has more incoming edges than lanes: the
            # code that fetches a second chunk is left out (its presence
            # alone cost 7 % on the 128^3 grid); a task that had more would
            # never turn ready and trip the watchdog
            *([] if self.single_chunk else self._gather_fetch_lines(indent + 2)),
            f"{pad}        _ready = _mb_next == _mb_end;",
            f"{pad}    }}",
            f"{pad}}}",
        ]

    def _mailbox_ready_lines(self, indent):
        """Readiness for the mailbox protocol: every incoming message has
        arrived.  A task's message slots are contiguous, in (source, position)
        order; lane ``l`` of the group polls slot ``next + l``; arrived
        messages are added to the task's own element in (source, position)
        order -- the order of the sequential loop -- by broadcasting them
        lane by lane, so the sum is deterministic."""
        pad = "    " * indent
        own = self._mailbox["register"]
        return [
            f"{pad}bool _ready = _mb_next == _mb_end;",
            f"{pad}if (!_ready) {{",
            f"{pad}    const int _mb_have = (_mb_end - _mb_next) < LCD_TASK_LANES ? "
            "(_mb_end - _mb_next) : LCD_TASK_LANES;",
            f"{pad}    const double _mb_value = _lane < _mb_have ? "
            "lcd_ld(&_lcd_mailbox[_mb_next + _lane]) : 0.0;",
            f"{pad}    int _mb_k = 0;",
            f"{pad}    for (; _mb_k < _mb_have; ++_mb_k) {{",
            f"{pad}        const double _mb_in = __shfl(_mb_value, _mb_k, LCD_TASK_LANES);",
            f"{pad}        if (lcd_is_empty(_mb_in)) break;",
            f"{pad}        {own} = {own} + _mb_in;",
            f"{pad}    }}",
            f"{pad}    _mb_next += _mb_k;",
            f"{pad}    _ready = _mb_next == _mb_end;",
            f"{pad}}}",
        ]

    def _pull_ready_lines(self, indent):
        """Readiness for the pull protocol: every producer this task reads
        from (the endpoint of the direct dependence over the mapped loop's
        range) has published ``done``."""
        pad = "    " * indent
        dependence = self.direct_dependence
        emitter = self._emitter
        loop = dependence.thread_loop
        lower, upper, _ = emitter.range_parts(loop)
        name = loop.target.id
        endpoint = emitter.expr(dependence.endpoint)
        guard = (emitter.expr(dependence.guard)
                 if dependence.guard is not None else "true")
        total = ("lcd_group_sum((double)_missing) != 0.0"
                 if self.task_lanes > 1 else "_missing != 0")
        return [
            f"{pad}int _missing = 0;",
            f"{pad}for ({name} = ({lower}) + _lane; {name} < {upper}; "
            f"{name} += LCD_TASK_LANES)",
            f"{pad}    if (({guard}) && lcd_load_relaxed(&done[{endpoint}]) == 0) "
            "{ _missing = 1; break; }",
            f"{pad}bool _ready = !({total});",
        ]

    def _stage_kernel_text(self, stage_name):
        """``_lcd_staged_k[s] = R[f(in_pos[s])]`` for every message ``s``."""
        gather = self._mailbox["gather"]
        emitter = self._emitter
        sources = []
        body = []
        for name, node, _ in gather["operands"]:
            if name not in gather["staged"]:
                continue
            for sub in ast.walk(node):
                if (isinstance(sub, ast.Name) and sub.id in self._kinds.arrays
                        and sub.id not in sources):
                    sources.append(sub.id)
            body.append(f"        {gather['staged'][name]}[t] = "
                        f"{emitter.expr(node)};")
        staged = list(gather["staged"].values())
        scalars = sorted({
            sub.id for name, node, _ in gather["operands"]
            if name in gather["staged"] for sub in ast.walk(node)
            if isinstance(sub, ast.Name) and sub.id in self._kinds.scalars
            and sub.id not in ("_g_pos",)})
        parameters = (
            [f"const LCD_T_{name}* __restrict__ {name}" for name in sources]
            + [f"LCD_T_{name} {name}" for name in scalars]
            + ["const int* __restrict__ _lcd_in_pos"]
            + [f"LCD_T_{name}* {name}" for name in staged]
            + ["long long count"])
        text = (f'\nextern "C" __global__ void {stage_name}('
                + ", ".join(parameters) + ")\n{\n"
                "    const long long t = (long long)blockIdx.x * blockDim.x + "
                "threadIdx.x;\n"
                "    if (t < count) {\n"
                "        const lcd_index_t _g_pos = _lcd_in_pos[t];\n"
                + "\n".join(body) + "\n    }\n}\n")
        return text, sources + scalars + ["_lcd_in_pos"] + staged

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
            if name == "task_count":
                continue
            launcher_arguments.append(name)
        args = []
        for name in kernel_arguments:
            if name in ("band_start", "band_end"):
                args.append("0")
            elif name == "task_count":
                args.append("_count")
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
            body.append(
                f"_hip.launch_levels({kernel_name!r}, band_ptr, "
                f"{max(1, self.threads_per_block // self.task_lanes)}, "
                f"{self.threads_per_block}, {call_args}, {start}, {end})")
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
            body.append(f"_count = _hip.length({count_array})")
            body.append(f"_hip.launch({reset_name!r}, ({reset_count} + 255) // 256 or 1, "
                        f"256, {reset_args})")
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
                 publish_values=True, look_ahead=True, segment_capacity=None):
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
        look_ahead=look_ahead, segment_capacity=segment_capacity)
    return lowerer.lower(code)

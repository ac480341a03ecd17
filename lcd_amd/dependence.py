"""Structural loop-carried dependence analysis for `@parallel` loops.

The reference derives ordering and reduction dependences with an SPF/Z3
pipeline (compiler/legality_check.py:406-470, compiler/dag_codegen.py:89-790)
and then projects them onto *edge rules* that the inspector enumerates.  Z3 is
not a dependency of this backend.  This module recognises, directly on the
Python AST, the access shapes that the reference's planner reduces the
supported solver loops to, and produces the same edge rules:

* a task writes its own element ``X[i]`` and other tasks read ``X[I[p]]`` for
  ``p`` in their own pointer segment           -> pull rule (source ``I[p]``,
  destination ``i``; SpTRSV-CSR, Gauss-Seidel; test_dag_codegen.py:58-70,
  test_gauss_seidel_codegen.py:143-148)
* a task updates ``X[I[p]] op= ...`` for ``p`` in its own segment and the owner
  reads ``X[i]``                               -> push rule (source ``i``,
  destination ``I[p]``; SpTRSV-CSC; test_dag_codegen.py:72-83) plus an atomic
  reduction on the update
* a task writes positions of its own segment ``D[p]`` and reads positions of
  the segment of ``I[q]``                      -> pull rule over ``q`` with
  the loop's ``break`` (ILU0-CSR; test_spilu0_codegen.py:129-144)
* a task reads or writes positions of the segments of every later task,
  ``for j in range(i + 1, n)``                 -> the relational rule
  ``i -> j`` for all later ``j``, plus the push rule over the own segment
  whose entries name the rows it updates there (ILU0-CSC;
  test_spilu0_codegen.py:146-150)

The analysis runs in the reference's three stages
(compiler/legality_check.py:172-383):

1. *candidates*: per array, the last write of every distinct access
   expression against the first read of every distinct access expression
   (plus the target of every associative augmented update, whose
   self-dependence must not be hidden by first-read filtering); a pair is a
   candidate when its index expressions differ or go through an index array.
   Statements are numbered S0, S1, ... over the function's assignments in
   source order, as the reference's frontend does (compiler/spf_raising.py:
   266-277).
2. *refutation*: the reference hands every candidate to Z3 with the
   ``function_props`` as axioms.  Here the structural facts are applied
   directly: different tasks own disjoint segments (monotone pointers); a
   task's own segment lies before every segment it visits through
   ``range(i + c, n)``; inside one sorted segment the entries below, at and
   above the owner's index are disjoint.  A self-dependence of an
   associative update becomes a reduction.
3. *projection*: every surviving dependence is mapped to an edge rule the
   inspector can enumerate.  A survivor that has no such rule is kept, as
   the reference keeps what its solver does not refute in time
   (compiler/legality_check.py:431-443): it is over-approximated by the
   chain ``i -> i + 1`` (:class:`NextRule`), whose closure is the complete
   order, unless ``strict=True`` asks for :class:`DependenceAnalysisError`
   instead.  Callers can also pass ``edge_rules=`` to the decorator.
"""

import ast
from copy import deepcopy
from dataclasses import dataclass, field

GUARD_NONE, GUARD_GREATER, GUARD_NOT_EQUAL = 0, 1, 2
ASSOCIATIVE_UPDATE_OPERATIONS = {
    ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.BitAnd: "&",
    ast.BitOr: "|", ast.BitXor: "^",
}


class DependenceAnalysisError(Exception):
    """The loop's cross-iteration dependences are outside the supported set."""


@dataclass(frozen=True)
class SegmentRule:
    """One inspector edge rule over a pointer-delimited segment.

    ``for seg in range(node_count): for p in range(ptr[seg] + lower_offset,
    ptr[seg + 1] + upper_offset): [if idx[p] >= seg: break]`` yields the edge
    ``seg -> idx[p]`` (``owner_is_source``) or ``idx[p] -> seg``.
    """

    pointer_array: str
    index_array: str
    owner_is_source: bool
    lower_offset: int = 0
    upper_offset: int = 0
    guard: int = GUARD_GREATER
    break_at_owner: bool = False
    block_iterator: str = "i"
    inner_iterator: str = "j"
    carried_by: str = ""

    @property
    def iterators(self):
        return [self.block_iterator, self.inner_iterator]

    def endpoint_source(self):
        return f"{self.index_array}[{self.inner_iterator}]"

    def describe(self):
        source, destination = (
            (self.block_iterator, self.endpoint_source())
            if self.owner_is_source
            else (self.endpoint_source(), self.block_iterator)
        )
        return (f"RAW on {self.carried_by}: {source} -> {destination} "
                f"over {self.inner_iterator} in segment of "
                f"{self.pointer_array}[{self.block_iterator}]")


@dataclass(frozen=True)
class LaterRule:
    """``for seg in range(node_count): for j in range(seg + lower_offset,
    node_count)`` yields the edge ``seg -> j``: the task touches segments of
    every later task, so all of them wait for it."""

    lower_offset: int = 1
    block_iterator: str = "i"
    inner_iterator: str = "j"
    carried_by: str = ""
    relation = 1

    @property
    def iterators(self):
        return [self.block_iterator, self.inner_iterator]

    def describe(self):
        return (f"RAW on {self.carried_by}: {self.block_iterator} -> "
                f"{self.inner_iterator} for every {self.inner_iterator} >= "
                f"{self.block_iterator} + {self.lower_offset}")


@dataclass(frozen=True)
class NextRule:
    """``seg -> seg + lower_offset``: with offset 1 the chain whose closure is
    the complete order, the safe over-approximation of a dependence that
    could be neither refuted nor enumerated."""

    lower_offset: int = 1
    block_iterator: str = "i"
    inner_iterator: str = "_lcd_next"
    carried_by: str = ""
    relation = 2

    @property
    def iterators(self):
        return [self.block_iterator, self.inner_iterator]

    def describe(self):
        return (f"RAW on {self.carried_by}: kept without an enumerable rule; "
                f"{self.block_iterator} -> {self.block_iterator} + "
                f"{self.lower_offset} (complete order)")


@dataclass(frozen=True)
class RawDependence:
    """One read-after-write candidate between two statements of the block
    loop and what became of it."""

    array: str
    from_statement_id: str        # the writer
    to_statement_id: str          # the reader
    write_index: str
    read_index: str
    kind: str = "RAW"             # "RAW" | "reduction"
    verdict: str = "kept"         # "kept" | "refuted"
    reason: str = ""
    rule: object = None           # SegmentRule | LaterRule | NextRule | None

    def __str__(self):
        return (f"{self.kind} on {self.array}: {self.from_statement_id}"
                f"[{self.write_index}] -> {self.to_statement_id}"
                f"[{self.read_index}] ({self.verdict}"
                f"{': ' + self.reason if self.reason else ''})")


@dataclass(frozen=True)
class ReductionSite:
    statement_id: str
    operator: str
    location: tuple
    array: str


@dataclass
class DependenceAnalysis:
    """``ordering_dependences`` holds the distinct edge rules (what the DAG
    planner consumes); ``raw_dependences`` every candidate with its verdict.
    The reference's ``analysis.ordering_dependences`` (one entry per
    dependence that survived its solver) corresponds to
    ``kept_dependences``, its ``reduction_dependences`` to
    ``reduction_candidates``."""

    ordering_dependences: list = field(default_factory=list)
    reduction_dependences: list = field(default_factory=list)
    reductions: dict = field(default_factory=dict)
    raw_dependences: list = field(default_factory=list)
    # reader-before-writer orderings kept beside the RAW ones (the reference
    # enumerates RAW only, compiler/legality_check.py:226-258): a task that
    # reads what a later task overwrites must come first here too
    war_dependences: list = field(default_factory=list)
    statement_ids: dict = field(default_factory=dict)   # (line, col) -> "Sk"
    conservative: bool = False    # a NextRule stands in for a kept candidate

    @property
    def kept_dependences(self):
        return [d for d in self.raw_dependences
                if d.verdict == "kept" and d.kind == "RAW"]

    @property
    def reduction_candidates(self):
        return [d for d in self.raw_dependences if d.kind == "reduction"]

    @property
    def atomic_statements(self):
        return list(self.reductions.values())


@dataclass(frozen=True)
class _Segment:
    """Positions ``[ptr[owner] + lower, ptr[owner + 1] + upper)``."""

    pointer_array: str
    owner: ast.expr
    lower_offset: int
    upper_offset: int
    lower_is_position: bool = False
    position_base: str = ""       # range(<position_base> + c, end)
    position_offset: int = 0


def _const_int(node):
    if isinstance(node, ast.Constant) and isinstance(node.value, int) and not (
            isinstance(node.value, bool)):
        return node.value
    if (isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub)
            and isinstance(node.operand, ast.Constant)
            and isinstance(node.operand.value, int)):
        return -node.operand.value
    return None


def _split_offset(node):
    """``expr + c`` / ``expr - c`` -> (expr, c)."""
    if isinstance(node, ast.BinOp) and isinstance(node.op, (ast.Add, ast.Sub)):
        right = _const_int(node.right)
        if right is not None:
            base, offset = _split_offset(node.left)
            return base, offset + (right if isinstance(node.op, ast.Add)
                                   else -right)
        left = _const_int(node.left)
        if left is not None and isinstance(node.op, ast.Add):
            base, offset = _split_offset(node.right)
            return base, offset + left
    return node, 0


def _same(a, b):
    return ast.dump(a) == ast.dump(b)


class _AliasTable:
    """Names assigned exactly once to a pure expression inside the function."""

    def __init__(self, function):
        counts = {}
        values = {}
        for node in ast.walk(function):
            targets = []
            if isinstance(node, ast.Assign):
                targets = node.targets
            elif isinstance(node, (ast.AugAssign, ast.AnnAssign)):
                targets = [node.target]
            elif isinstance(node, ast.For):
                targets = [node.target]
            for target in targets:
                for name in ast.walk(target):
                    if isinstance(name, ast.Name) and isinstance(
                            name.ctx, ast.Store):
                        counts[name.id] = counts.get(name.id, 0) + 1
                        if isinstance(node, ast.Assign) and len(
                                node.targets) == 1 and isinstance(
                                    node.targets[0], ast.Name):
                            values[name.id] = node.value
        self.values = {
            name: value for name, value in values.items()
            if counts.get(name) == 1 and not any(
                isinstance(n, ast.Call) for n in ast.walk(value))
        }

    def resolve(self, node, depth=0):
        """Substitute aliases everywhere inside ``node`` (a copy is returned)."""
        if depth > 16:
            return node
        table = self

        class Substitute(ast.NodeTransformer):
            def visit_Name(self, name):
                if isinstance(name.ctx, ast.Load) and name.id in table.values:
                    return table.resolve(table.values[name.id], depth + 1)
                return name

        return Substitute().visit(deepcopy(node))


def pointer_arrays(function_props):
    return [
        name for name, properties in (function_props or {}).items()
        if isinstance(name, str) and "monotonically_increasing" in properties
    ]


def find_block_loop(function, block_iterator):
    matches = [
        node for node in ast.walk(function)
        if isinstance(node, ast.For) and isinstance(node.target, ast.Name)
        and node.target.id == block_iterator
    ]
    if len(matches) != 1:
        raise DependenceAnalysisError(
            f"Expected exactly one loop over {block_iterator!r}; "
            f"found {len(matches)}.")
    return matches[0]


def sorted_segment_pairs(function_props):
    """(pointer array, index array) pairs whose segments are sorted
    (``segmented_monotonically_increasing``)."""
    pairs = set()
    for key, properties in (function_props or {}).items():
        if not (isinstance(key, tuple) and len(key) == 2):
            continue
        for entry in properties:
            name = entry[0] if isinstance(entry, (tuple, list)) else entry
            if name == "segmented_monotonically_increasing":
                pairs.add(tuple(key))
    return pairs


def triangular_pairs(function_props):
    """(pointer array, index array) pairs with the ``triangularity``
    property: every position behind a segment's first holds an index above
    the segment's owner (compiler/SMT_Generator.py:309-310)."""
    return {tuple(key) for key, properties in (function_props or {}).items()
            if isinstance(key, tuple) and len(key) == 2
            and "triangularity" in [entry[0] if isinstance(entry, (tuple, list))
                                    else entry for entry in properties]}


def number_statements(function):
    """S0, S1, ... for the assignments of ``function`` in source order
    (compiler/spf_raising.py:266-277): (line, column) -> id."""
    found = sorted(
        (node.lineno, node.col_offset) for node in ast.walk(function)
        if isinstance(node, (ast.Assign, ast.AugAssign, ast.AnnAssign)))
    return {location: f"S{k}" for k, location in enumerate(found)}


def unique_loop_iterators(function, block_iterator):
    """A copy of ``function`` in which every ``for`` loop binds a name of its
    own: a loop that binds a name an earlier loop has bound gets a fresh one
    (``p`` -> ``p__2``), in its body and in everything that follows it in
    program order until the name is bound again.  The analysis keeps what it
    knows of a loop (its range, its break tests, the value its search
    matches) under the iterator's name, and two accesses spelled alike are
    the same element of the same iteration only when the same loop binds
    their iterator; with one name per loop both hold by construction.  The
    block iterator keeps its name, and so does the first loop over each other
    name (the thread-mapped loop is found by its name later)."""
    function = deepcopy(function)
    bound, counter = set(), {}

    class Rename(ast.NodeTransformer):
        def __init__(self, mapping):
            self.mapping = mapping

        def visit_Name(self, node):
            if node.id in self.mapping:
                return ast.copy_location(
                    ast.Name(id=self.mapping[node.id], ctx=node.ctx), node)
            return node

    def walk(statements, mapping):
        for statement in statements:
            if isinstance(statement, ast.For):
                statement.iter = Rename(mapping).visit(statement.iter)
                target = statement.target
                if isinstance(target, ast.Name):
                    name = target.id
                    if name != block_iterator and name in bound:
                        counter[name] = counter.get(name, 1) + 1
                        mapping[name] = f"{name}__{counter[name]}"
                    else:
                        mapping.pop(name, None)
                    bound.add(name)
                    statement.target = Rename(mapping).visit(target)
                else:
                    statement.target = Rename(mapping).visit(target)
                walk(statement.body, mapping)
                walk(statement.orelse, mapping)
            elif isinstance(statement, (ast.If, ast.While)):
                statement.test = Rename(mapping).visit(statement.test)
                walk(statement.body, mapping)
                walk(statement.orelse, mapping)
            else:
                Rename(mapping).visit(statement)

    walk(function.body, {})
    return function


class _Analyzer:
    def __init__(self, function, block_iterator, function_props,
                 strict=False):
        function = unique_loop_iterators(function, block_iterator)
        self.function = function
        self.block = block_iterator
        self.strict = strict
        self.sorted_pairs = sorted_segment_pairs(function_props)
        self.triangular = triangular_pairs(function_props)
        self.statement_ids = number_statements(function)
        self.current_statement = None
        self.aliases = _AliasTable(function)
        self.pointers = set(pointer_arrays(function_props))
        self.segments = {}     # iterator -> _Segment
        self.later = {}        # iterator over range(block + c, count) -> c
        self.needles = {}      # segment iterator -> value its search matches
        self.node_count = None
        self.breaks = {}       # iterator -> list of resolved break tests
        self.writes = []       # (array, classification, node, is_update)
        self.reads = []        # (array, classification)
        self.reductions = {}
        self.statement_counter = 0

    # ---- loop ranges ----------------------------------------------------
    def _segment_of_range(self, loop):
        call = loop.iter
        if not (isinstance(call, ast.Call) and isinstance(call.func, ast.Name)
                and call.func.id == "range" and len(call.args) == 2):
            return None
        lower = self.aliases.resolve(call.args[0])
        upper = self.aliases.resolve(call.args[1])
        lower_base, lower_offset = _split_offset(lower)
        upper_base, upper_offset = _split_offset(upper)
        if not (isinstance(upper_base, ast.Subscript)
                and isinstance(upper_base.value, ast.Name)
                and upper_base.value.id in self.pointers):
            return None
        pointer = upper_base.value.id
        owner_plus, one = _split_offset(upper_base.slice)
        if one != 1:
            return None
        if (isinstance(lower_base, ast.Subscript)
                and isinstance(lower_base.value, ast.Name)
                and lower_base.value.id == pointer
                and _same(lower_base.slice, owner_plus)):
            return _Segment(pointer, owner_plus, lower_offset, upper_offset)
        # lower bound is a position of the same segment plus a constant
        if isinstance(lower_base, ast.Name) and lower_base.id in self.segments:
            outer = self.segments[lower_base.id]
            if (outer.pointer_array == pointer
                    and _same(outer.owner, owner_plus) and lower_offset >= 0):
                return _Segment(pointer, owner_plus, outer.lower_offset,
                                upper_offset, lower_is_position=True,
                                position_base=lower_base.id,
                                position_offset=lower_offset)
        return None

    # ---- access classification -------------------------------------------
    def _owner_kind(self, owner):
        owner = self.aliases.resolve(owner)
        if isinstance(owner, ast.Name) and owner.id == self.block:
            return ("self",)
        if isinstance(owner, ast.Name) and owner.id in self.later:
            return ("later", owner.id)
        if (isinstance(owner, ast.Subscript) and isinstance(owner.value, ast.Name)
                and isinstance(owner.slice, ast.Name)
                and owner.slice.id in self.segments):
            inner = self.segments[owner.slice.id]
            if self._owner_kind(inner.owner) == ("self",):
                return ("indirect", owner.value.id, owner.slice.id)
        return ("unknown", ast.unparse(owner))

    def _classify(self, index):
        index = self.aliases.resolve(index)
        if isinstance(index, ast.Name) and index.id == self.block:
            return ("self",)
        if isinstance(index, ast.Name) and index.id in self.segments:
            kind = self._owner_kind(self.segments[index.id].owner)
            if kind == ("self",):
                return ("own_position", index.id)
            if kind[0] == "indirect":
                return ("other_position", kind[1], kind[2], index.id)
            if kind[0] == "later":
                return ("later_position", kind[1], index.id)
            return ("unknown", ast.unparse(index))
        if isinstance(index, ast.Subscript) and isinstance(index.value, ast.Name):
            base, offset = _split_offset(index.slice)
            if (isinstance(base, ast.Name) and base.id in self.segments
                    and offset == 0
                    and self._owner_kind(self.segments[base.id].owner)
                    == ("self",)):
                return ("indirect", index.value.id, base.id)
        return ("unknown", ast.unparse(index))

    def _later_offset(self, loop):
        """``c`` when ``loop`` is ``for j in range(block + c, node_count)``
        with ``c >= 1``, else None."""
        call = loop.iter
        if not (isinstance(call, ast.Call) and isinstance(call.func, ast.Name)
                and call.func.id == "range" and len(call.args) == 2
                and self.node_count is not None):
            return None
        base, offset = _split_offset(self.aliases.resolve(call.args[0]))
        if not (isinstance(base, ast.Name) and base.id == self.block
                and offset >= 1):
            return None
        if not _same(self.aliases.resolve(call.args[1]), self.node_count):
            return None
        return offset

    def _search_needle(self, loop):
        """The value ``v`` of ``for p in <segment>: if I[p] == v: ...``."""
        if not (len(loop.body) == 1 and isinstance(loop.body[0], ast.If)
                and isinstance(loop.body[0].test, ast.Compare)
                and len(loop.body[0].test.ops) == 1
                and isinstance(loop.body[0].test.ops[0], ast.Eq)):
            return None
        test = loop.body[0].test
        for entry, other in ((test.left, test.comparators[0]),
                             (test.comparators[0], test.left)):
            if (isinstance(entry, ast.Subscript)
                    and isinstance(entry.slice, ast.Name)
                    and entry.slice.id == loop.target.id):
                return self.aliases.resolve(other)
        return None

    # ---- traversal ---------------------------------------------------------
    def _record_reads(self, node, written_arrays):
        for sub in ast.walk(node):
            if (isinstance(sub, ast.Subscript) and isinstance(sub.ctx, ast.Load)
                    and isinstance(sub.value, ast.Name)
                    and sub.value.id in written_arrays):
                self.reads.append((sub.value.id, self._classify(sub.slice),
                                   sub, self.current_statement))

    def _visit(self, statements, written_arrays, loop_stack):
        for statement in statements:
            if not isinstance(statement, (ast.Assign, ast.AugAssign)):
                self.current_statement = None
            if isinstance(statement, ast.For):
                segment = None
                if isinstance(statement.target, ast.Name):
                    segment = self._segment_of_range(statement)
                    if segment is not None:
                        self.segments[statement.target.id] = segment
                        needle = self._search_needle(statement)
                        if needle is not None:
                            self.needles[statement.target.id] = needle
                    else:
                        offset = self._later_offset(statement)
                        if offset is not None:
                            self.later[statement.target.id] = offset
                self._record_reads(statement.iter, written_arrays)
                self._visit(statement.body, written_arrays,
                            loop_stack + [statement])
            elif isinstance(statement, ast.If):
                self._record_reads(statement.test, written_arrays)
                if (loop_stack and len(statement.body) == 1
                        and isinstance(statement.body[0], ast.Break)
                        and not statement.orelse
                        and isinstance(loop_stack[-1].target, ast.Name)):
                    self.breaks.setdefault(
                        loop_stack[-1].target.id, []
                    ).append(self.aliases.resolve(statement.test))
                self._visit(statement.body, written_arrays, loop_stack)
                self._visit(statement.orelse, written_arrays, loop_stack)
            elif isinstance(statement, ast.While):
                self._record_reads(statement.test, written_arrays)
                self._visit(statement.body, written_arrays, loop_stack)
            elif isinstance(statement, ast.Assign):
                self.current_statement = statement
                self._record_reads(statement.value, written_arrays)
                for target in statement.targets:
                    if isinstance(target, ast.Subscript) and isinstance(
                            target.value, ast.Name):
                        self._record_reads(target.slice, written_arrays)
                        self.writes.append((
                            target.value.id, self._classify(target.slice),
                            statement, False))
            elif isinstance(statement, ast.AugAssign):
                self.current_statement = statement
                self._record_reads(statement.value, written_arrays)
                target = statement.target
                if isinstance(target, ast.Subscript) and isinstance(
                        target.value, ast.Name):
                    self._record_reads(target.slice, written_arrays)
                    if target.value.id in written_arrays:
                        # an update reads its own target
                        self.reads.append((
                            target.value.id, self._classify(target.slice),
                            target, statement))
                    self.writes.append((
                        target.value.id, self._classify(target.slice),
                        statement, True))
            elif isinstance(statement, ast.Expr):
                self._record_reads(statement.value, written_arrays)

    def _break_at_owner(self, iterator, index_array):
        """True when the loop over ``iterator`` starts with
        ``if index_array[iterator] >= block: break``."""
        for test in self.breaks.get(iterator, []):
            if (isinstance(test, ast.Compare) and len(test.ops) == 1
                    and isinstance(test.ops[0], ast.GtE)
                    and isinstance(test.left, ast.Subscript)
                    and isinstance(test.left.value, ast.Name)
                    and test.left.value.id == index_array
                    and isinstance(test.left.slice, ast.Name)
                    and test.left.slice.id == iterator
                    and isinstance(test.comparators[0], ast.Name)
                    and test.comparators[0].id == self.block):
                return True
        if self.breaks.get(iterator):
            raise DependenceAnalysisError(
                f"Unsupported break condition in the loop over {iterator!r}.")
        return False

    def _rule(self, owner_is_source, index_array, iterator, array):
        segment = self.segments[iterator]
        if segment.lower_is_position:
            raise DependenceAnalysisError(
                f"The dependence carried by {array!r} is enumerated by a loop "
                f"over {iterator!r} whose lower bound is not a segment start.")
        broken = self._break_at_owner(iterator, index_array)
        if broken and owner_is_source:
            raise DependenceAnalysisError(
                "A break-guarded segment loop cannot release successors.")
        return SegmentRule(
            pointer_array=segment.pointer_array,
            index_array=index_array,
            owner_is_source=owner_is_source,
            lower_offset=segment.lower_offset,
            upper_offset=segment.upper_offset,
            guard=GUARD_NONE if broken else GUARD_GREATER,
            break_at_owner=broken,
            block_iterator=self.block,
            inner_iterator=iterator,
            carried_by=array,
        )

    def _later_rule(self, iterator, array):
        return LaterRule(lower_offset=self.later[iterator],
                         block_iterator=self.block, inner_iterator=iterator,
                         carried_by=array)

    def _row_rule(self, write_kind, read_kind, array):
        """Two tasks meet in a later task's segment: the writer at the entry
        its search finds for ``I[q]`` (``q`` in its own segment), the reader
        at the entry found for its own id.  They coincide when ``I[q]`` is
        the reader: the push rule over ``q``."""
        written = self.needles.get(write_kind[2])
        read = self.needles.get(read_kind[2])
        if written is None or read is None:
            return None
        if not (isinstance(read, ast.Name) and read.id == self.block):
            return None
        kind = self._classify(written) if isinstance(
            written, ast.Subscript) else ("unknown",)
        if kind[0] != "indirect":
            return None
        return self._rule(True, kind[1], kind[2], array)

    # ---- column classes inside one sorted segment -----------------------
    def _index_array_of(self, iterator):
        """The index array whose entries the loop over ``iterator`` tests
        (break test or search needle), if any."""
        for test in self.breaks.get(iterator, []):
            if (isinstance(test, ast.Compare)
                    and isinstance(test.left, ast.Subscript)
                    and isinstance(test.left.value, ast.Name)):
                return test.left.value.id
        return None

    def _own_class(self, iterator):
        """Where the entry at an own-segment position lies relative to the
        task's index: "below" when the loop leaves at the first entry that
        is not below it (``if I[p] >= i: break`` on a sorted segment)."""
        segment = self.segments.get(iterator)
        if segment is None or segment.lower_is_position:
            return "any"
        index_array = self._index_array_of(iterator)
        if index_array is None or (segment.pointer_array,
                                   index_array) not in self.sorted_pairs:
            return "any"
        try:
            return "below" if self._break_at_owner(iterator, index_array) \
                else "any"
        except DependenceAnalysisError:
            return "any"

    def _other_class(self, index_array, outer, iterator):
        """Where the entry found by the search loop over ``iterator`` (in the
        segment of ``index_array[outer]``) lies relative to that segment's
        owner: "diag" when the search matches the owner itself, "above" when
        it matches a later entry of the sorted own segment than the owner's
        (``range(outer + c, end)`` with ``c >= 1``)."""
        needle = self.needles.get(iterator)
        if needle is None:
            return "any"
        owner = self.aliases.resolve(self.segments[iterator].owner)
        if _same(needle, owner):
            return "diag"
        if (isinstance(needle, ast.Subscript)
                and isinstance(needle.value, ast.Name)
                and needle.value.id == index_array
                and isinstance(needle.slice, ast.Name)):
            later = self.segments.get(needle.slice.id)
            if (later is not None and later.lower_is_position
                    and later.position_base == outer
                    and later.position_offset >= 1
                    and (later.pointer_array, index_array) in self.sorted_pairs):
                return "above"
        return "any"

    # ---- stage 2 and 3 for one candidate --------------------------------
    def _decide(self, array, write_kind, read_kind, statement, is_update,
                same_statement):
        """(verdict, reason, rule, kind) of one write/read pair."""
        own = ("self", "own_position")
        if write_kind[0] == "unknown" or read_kind[0] == "unknown":
            which = write_kind if write_kind[0] == "unknown" else read_kind
            return ("kept", f"index {which[1]} is not a recognised shape",
                    None, "RAW")
        if write_kind[0] == "indirect" and read_kind[0] == "indirect":
            if same_statement and is_update and type(
                    statement.op) in ASSOCIATIVE_UPDATE_OPERATIONS:
                return ("kept", "associative update of a shared element",
                        None, "reduction")
            return ("refuted", "read-modify-write of the update itself", None,
                    "RAW")
        if write_kind[0] in own and read_kind[0] in own:
            return ("refuted", "different tasks own disjoint segments", None,
                    "RAW")
        if write_kind[0] in own and read_kind[0] == "later_position":
            return ("refuted", "the segments a task visits through "
                    "range(i + c, n) lie behind the reader, the writer's own "
                    "segment before it", None, "RAW")
        if write_kind == ("self",) and read_kind[0] == "indirect":
            segment = self.segments[read_kind[2]]
            if ((segment.pointer_array, read_kind[1]) in self.triangular
                    and segment.lower_offset >= 1):
                return ("refuted", "the entries behind a segment's first lie "
                        "above the reader's index (triangularity), the "
                        "writer's below it", None, "RAW")
            return ("kept", "", self._rule(False, read_kind[1], read_kind[2],
                                           array), "RAW")
        if write_kind[0] == "indirect" and read_kind == ("self",):
            return ("kept", "", self._rule(True, write_kind[1], write_kind[2],
                                           array), "RAW")
        if write_kind[0] == "own_position" and read_kind[0] == "other_position":
            written = self._own_class(write_kind[1])
            read = self._other_class(read_kind[1], read_kind[2], read_kind[3])
            if "any" not in (written, read) and written != read:
                return ("refuted", f"entries {written} the owner's index are "
                        f"written, the entry {read} it is read", None, "RAW")
            return ("kept", "", self._rule(False, read_kind[1], read_kind[2],
                                           array), "RAW")
        if write_kind[0] == "later_position" and read_kind[0] == "later_position":
            rule = self._row_rule(write_kind, read_kind, array)
            if rule is None:
                return ("kept", "two later segments meet at entries that "
                        "cannot be enumerated", None, "RAW")
            return ("kept", "", rule, "RAW")
        if write_kind[0] == "later_position" and read_kind[0] in own:
            return ("kept", "", self._later_rule(write_kind[1], array), "RAW")
        return ("kept", f"write {write_kind[0]} / read {read_kind[0]} has no "
                "enumerable rule", None, "RAW")

    def _anti_rule(self, array, write_kind, read_kind):
        """The rule that keeps a reader ahead of the later task that
        overwrites what it reads, for the two shapes whose RAW direction is
        refuted because the element lies BEHIND the reader: a read of the
        segments of ``range(i + c, n)`` against a write of the own segment
        (reader i before every task it visits), and a read of ``X[I[p]]``
        over a triangular segment against a write of ``X[i]`` (reader i
        before task ``I[p]``).  None for every other pair."""
        own = ("self", "own_position")
        if write_kind[0] in own and read_kind[0] == "later_position":
            return self._later_rule(read_kind[1], array)
        if write_kind == ("self",) and read_kind[0] == "indirect":
            segment = self.segments[read_kind[2]]
            if ((segment.pointer_array, read_kind[1]) in self.triangular
                    and segment.lower_offset >= 1
                    and not segment.lower_is_position):
                try:
                    return self._rule(True, read_kind[1], read_kind[2], array)
                except DependenceAnalysisError:
                    return None
        return None

    def run(self):
        loop = find_block_loop(self.function, self.block)
        if (isinstance(loop.iter, ast.Call) and loop.iter.args
                and not loop.iter.keywords):
            self.node_count = self.aliases.resolve(loop.iter.args[-1])
        written_arrays = set()
        for node in ast.walk(loop):
            target = None
            if isinstance(node, ast.Assign):
                for candidate in node.targets:
                    if isinstance(candidate, ast.Subscript):
                        target = candidate
            elif isinstance(node, ast.AugAssign) and isinstance(
                    node.target, ast.Subscript):
                target = node.target
            if target is not None and isinstance(target.value, ast.Name):
                written_arrays.add(target.value.id)
        self._visit(loop.body, written_arrays, [loop])

        def sid(statement):
            if statement is None:
                return "-"
            return self.statement_ids.get(
                (statement.lineno, statement.col_offset), "-")

        def text(node):
            return ast.unparse(node.slice if isinstance(node, ast.Subscript)
                               else node)

        def indirect(node):
            index = node.slice if isinstance(node, ast.Subscript) else node
            return any(isinstance(sub, ast.Subscript)
                       for sub in ast.walk(self.aliases.resolve(index)))

        # stage 1: last write and first read of every access expression
        last_writes = {}
        for array, kind, statement, is_update in self.writes:
            target = (statement.target if isinstance(statement, ast.AugAssign)
                      else next(t for t in statement.targets
                                if isinstance(t, ast.Subscript)
                                and t.value.id == array))
            last_writes[(array, text(target))] = (
                array, kind, statement, is_update, target)
        first_reads, update_reads = {}, []
        for array, kind, node, statement in self.reads:
            key = (array, text(node))
            own_target = (isinstance(statement, ast.AugAssign)
                          and node is statement.target)
            if own_target:
                if type(statement.op) in ASSOCIATIVE_UPDATE_OPERATIONS:
                    update_reads.append((array, kind, node, statement))
                if key not in first_reads:
                    first_reads[key] = (array, kind, node, statement)
                continue
            first_reads.setdefault(key, (array, kind, node, statement))
        selected = list(first_reads.values())
        chosen = {(id(statement), array, text(node))
                  for array, _, node, statement in selected}
        selected += [read for read in update_reads
                     if (id(read[3]), read[0], text(read[2])) not in chosen]

        # scattered plain writes cannot be ordered by any rule
        reductions, reduction_rules = {}, []
        for array, kind, statement, is_update, _ in last_writes.values():
            if kind[0] == "other_position":
                raise DependenceAnalysisError(
                    f"{ast.unparse(statement)!r} writes another task's "
                    "segment; this pattern is not supported.")
            if kind[0] == "indirect":
                operator = ASSOCIATIVE_UPDATE_OPERATIONS.get(
                    type(statement.op)) if is_update else None
                if operator is None:
                    raise DependenceAnalysisError(
                        f"{ast.unparse(statement)!r} scatters a "
                        "non-associative write to other tasks' elements.")
                location = (statement.lineno, statement.col_offset)
                if location not in reductions:
                    reductions[location] = ReductionSite(
                        statement_id=f"S{len(reductions) + 1}",
                        operator=operator, location=location, array=array)
                    reduction_rules.append(
                        f"reduction on {array}[{kind[1]}[{kind[2]}]] "
                        f"({operator}=)")

        # stages 2 and 3
        raw, war, rules, conservative = [], [], [], False
        for array, write_kind, statement, is_update, target in (
                last_writes.values()):
            for read_array, read_kind, node, reader in selected:
                if read_array != array:
                    continue
                if text(node) == text(target) and not indirect(node):
                    continue        # the same element of the same iteration
                verdict, reason, rule, kind = self._decide(
                    array, write_kind, read_kind, statement, is_update,
                    reader is statement)
                if verdict == "kept" and kind == "RAW" and rule is None:
                    if self.strict:
                        raise DependenceAnalysisError(
                            f"Unsupported dependence on {array!r} between "
                            f"{ast.unparse(statement)!r} and the read "
                            f"{array}[{text(node)}]: {reason}.")
                    rule = NextRule(block_iterator=self.block,
                                    carried_by=array)
                    conservative = True
                raw.append(RawDependence(
                    array=array, from_statement_id=sid(statement),
                    to_statement_id=sid(reader), write_index=text(target),
                    read_index=text(node), kind=kind, verdict=verdict,
                    reason=reason, rule=rule))
                if rule is not None and rule not in rules:
                    rules.append(rule)
                if verdict == "refuted":
                    anti = self._anti_rule(array, write_kind, read_kind)
                    if anti is not None:
                        war.append(RawDependence(
                            array=array, from_statement_id=sid(reader),
                            to_statement_id=sid(statement),
                            write_index=text(target), read_index=text(node),
                            kind="WAR", verdict="kept",
                            reason="the reader comes before the task that "
                                   "overwrites the element", rule=anti))
                        if anti not in rules:
                            rules.append(anti)
        if any(isinstance(rule, NextRule) for rule in rules):
            # the chain already orders everything
            rules = [rule for rule in rules if isinstance(rule, NextRule)][:1]
        rules.sort(key=lambda rule: isinstance(rule, (LaterRule, NextRule)))
        return DependenceAnalysis(
            ordering_dependences=rules,
            reduction_dependences=reduction_rules,
            reductions=reductions,
            raw_dependences=raw,
            war_dependences=war,
            statement_ids=dict(self.statement_ids),
            conservative=conservative,
        )


def analyze_dependences(function_ast, block_iterator, function_props=None,
                        strict=False):
    """Return the :class:`DependenceAnalysis` of the block loop.

    ``function_ast`` is an ``ast.Module`` holding one function, or the
    ``ast.FunctionDef`` itself.  ``strict=True`` raises
    :class:`DependenceAnalysisError` for a dependence that has no
    enumerable edge rule instead of keeping it as the complete order.
    """
    function = function_ast
    if isinstance(function_ast, ast.Module):
        functions = [n for n in function_ast.body
                     if isinstance(n, ast.FunctionDef)]
        if len(functions) != 1:
            raise DependenceAnalysisError("Expected exactly one function.")
        function = functions[0]
    return _Analyzer(function, block_iterator, function_props, strict).run()

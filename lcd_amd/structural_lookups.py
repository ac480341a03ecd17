"""Structure-only sparse searches hoisted into the inspector.

A loop that looks for the entry ``indices[p] == segment`` inside the segment
``[pointer[segment], pointer[segment + 1])`` (the diagonal search of ILU0)
depends on the sparsity structure only.  The plan records one position table
per (pointer, index) array pair; the table is built on the device by
``lcdhip_lookup_build`` and the kernel reads ``table[segment]`` instead of
searching.  Mirrors compiler/structural_lookups.py of the reference
(plan :55-105, materialisation :108-124/279-333, rewrite :127-177), with the
materialisation moved to the GPU.
"""

import ast
from copy import deepcopy
from dataclasses import dataclass

import numpy as np

SEGMENTED_MONOTONIC = "segmented_monotonically_increasing"
LOOKUP_NAME_PREFIX = "_lcd_lookup_position_"


class StructuralLookupError(Exception):
    """Concrete inputs violate a structural lookup plan."""


@dataclass(frozen=True)
class StructuralLookup:
    name: str
    pointer_array: str
    index_array: str
    sorted_segments: bool = False

    @property
    def argument_names(self):
        return self.pointer_array, self.index_array


@dataclass(frozen=True)
class SearchMatch:
    """``for it in range(ptr[seg], ptr[seg+1]): if idx[it] == needle: body;
    break``."""

    iterator: str
    segment: ast.expr
    needle: ast.expr
    matched_body: tuple
    pointer_array: str
    index_array: str


def property_name(entry):
    if isinstance(entry, (tuple, list)) and entry:
        return entry[0]
    return entry


def segmented_array_pairs(function_props):
    pairs = []
    for key, properties in (function_props or {}).items():
        if (isinstance(key, tuple) and len(key) == 2
                and all(isinstance(name, str) for name in key)
                and any(property_name(p) == SEGMENTED_MONOTONIC
                        for p in properties)):
            if (key[0], key[1]) not in pairs:
                pairs.append((key[0], key[1]))
    return pairs


def _subscript_of(node, array):
    return (isinstance(node, ast.Subscript) and isinstance(node.value, ast.Name)
            and node.value.id == array)


def structure_aliases(function_ast):
    """Names assigned exactly once to an expression over arrays that the
    function never stores to (``col_start = A_indptr[k]``): a search whose
    bounds are such names is the same search as one over the expressions
    (the reference normalises these aliases away before matching,
    compiler/ast_normalization.py:7-30)."""
    stored_arrays, counts, values = set(), {}, {}
    for node in ast.walk(function_ast):
        if isinstance(node, ast.Subscript) and isinstance(
                node.ctx, ast.Store) and isinstance(node.value, ast.Name):
            stored_arrays.add(node.value.id)
        if isinstance(node, ast.arg):
            counts[node.arg] = counts.get(node.arg, 0) + 2
        if isinstance(node, ast.Name) and isinstance(node.ctx, ast.Store):
            counts[node.id] = counts.get(node.id, 0) + 1
        if (isinstance(node, ast.Assign) and len(node.targets) == 1
                and isinstance(node.targets[0], ast.Name)):
            values[node.targets[0].id] = node.value
    aliases = {}
    for name, value in values.items():
        if counts.get(name) != 1:
            continue
        parts = list(ast.walk(value))
        if any(isinstance(part, (ast.Call, ast.Attribute)) for part in parts):
            continue
        if any(isinstance(part, ast.Subscript)
               and not (isinstance(part.value, ast.Name)
                        and part.value.id not in stored_arrays)
               for part in parts):
            continue
        if not any(isinstance(part, ast.Subscript) for part in parts):
            continue
        aliases[name] = value
    return aliases


def _resolve(node, aliases):
    if isinstance(node, ast.Name) and aliases and node.id in aliases:
        return aliases[node.id]
    return node


def match_segment_search(node, array_pairs, aliases=None):
    """Recognise the canonical equality search over one segment."""
    if not (isinstance(node, ast.For) and not node.orelse
            and isinstance(node.target, ast.Name)
            and isinstance(node.iter, ast.Call)
            and isinstance(node.iter.func, ast.Name)
            and node.iter.func.id == "range" and len(node.iter.args) == 2
            and not node.iter.keywords and len(node.body) == 1
            and isinstance(node.body[0], ast.If)):
        return None
    branch = node.body[0]
    if (branch.orelse or not branch.body
            or not isinstance(branch.body[-1], ast.Break)
            or not isinstance(branch.test, ast.Compare)
            or len(branch.test.ops) != 1
            or not isinstance(branch.test.ops[0], ast.Eq)):
        return None
    iterator = node.target.id
    lower, upper = (_resolve(bound, aliases) for bound in node.iter.args)
    left, right = branch.test.left, branch.test.comparators[0]
    for pointer_array, index_array in array_pairs:
        if not (_subscript_of(lower, pointer_array)
                and _subscript_of(upper, pointer_array)):
            continue
        expected = ast.BinOp(left=deepcopy(lower.slice), op=ast.Add(),
                             right=ast.Constant(value=1))
        if ast.dump(upper.slice) != ast.dump(expected):
            continue

        def is_lookup(side):
            return (_subscript_of(side, index_array)
                    and isinstance(side.slice, ast.Name)
                    and side.slice.id == iterator)

        if is_lookup(left):
            needle = right
        elif is_lookup(right):
            needle = left
        else:
            continue
        if any(isinstance(n, ast.Name) and n.id == iterator
               for n in ast.walk(needle)):
            continue
        return SearchMatch(
            iterator=iterator, segment=deepcopy(lower.slice),
            needle=deepcopy(needle),
            matched_body=tuple(deepcopy(branch.body[:-1])),
            pointer_array=pointer_array, index_array=index_array)
    return None


def _self_lookup(match):
    return ast.dump(match.needle) == ast.dump(match.segment)


def create_structural_lookup_plan(function_ast, function_props=None):
    """One table per array pair that has a self-segment search."""
    array_pairs = segmented_array_pairs(function_props)
    if not array_pairs:
        return ()
    used = {n.id for n in ast.walk(function_ast) if isinstance(n, ast.Name)}
    planned = []
    aliases = structure_aliases(function_ast)
    for node in ast.walk(function_ast):
        match = match_segment_search(node, array_pairs, aliases)
        if match is None or not _self_lookup(match):
            continue
        pair = (match.pointer_array, match.index_array)
        if pair not in planned:
            planned.append(pair)
    plan = []
    for position, (pointer_array, index_array) in enumerate(planned):
        suffix = position
        name = f"{LOOKUP_NAME_PREFIX}{suffix}"
        while name in used:
            suffix += 1
            name = f"{LOOKUP_NAME_PREFIX}{suffix}"
        used.add(name)
        plan.append(StructuralLookup(name, pointer_array, index_array, True))
    return tuple(plan)


def structural_argument_names(plan):
    names = []
    for lookup in plan or ():
        for name in lookup.argument_names:
            if name not in names:
                names.append(name)
    return names


def structural_lookup_names(plan):
    return [lookup.name for lookup in plan or ()]


def rewrite_structural_lookups(function_ast, plan, function_props=None):
    """Replace planned searches by ``it = table[segment]; if it >= 0: body``."""
    if not plan:
        return deepcopy(function_ast)
    array_pairs = segmented_array_pairs(function_props)
    by_pair = {(l.pointer_array, l.index_array): l for l in plan}
    aliases = structure_aliases(function_ast)

    class Rewriter(ast.NodeTransformer):
        def visit_For(self, node):
            node = self.generic_visit(node)
            match = match_segment_search(node, array_pairs, aliases)
            if match is None or not _self_lookup(match):
                return node
            lookup = by_pair.get((match.pointer_array, match.index_array))
            if lookup is None:
                return node
            position = ast.Assign(
                targets=[ast.Name(id=match.iterator, ctx=ast.Store())],
                value=ast.Subscript(
                    value=ast.Name(id=lookup.name, ctx=ast.Load()),
                    slice=deepcopy(match.segment), ctx=ast.Load()))
            found = ast.If(
                test=ast.Compare(
                    left=ast.Name(id=match.iterator, ctx=ast.Load()),
                    ops=[ast.GtE()], comparators=[ast.Constant(value=0)]),
                body=[deepcopy(s) for s in match.matched_body] or [ast.Pass()],
                orelse=[])
            return [ast.copy_location(position, node),
                    ast.copy_location(found, node)]

    return ast.fix_missing_locations(Rewriter().visit(deepcopy(function_ast)))


def validate_lookup_arrays(lookup, pointers, indices):
    """Host-side shape/dtype checks that need no array contents."""
    pointers, indices = np.asarray(pointers), np.asarray(indices)
    if pointers.ndim != 1 or indices.ndim != 1:
        raise StructuralLookupError(
            f"{lookup.pointer_array} and {lookup.index_array} must be 1-D.")
    if pointers.size == 0:
        raise StructuralLookupError(
            f"{lookup.pointer_array} must contain at least one offset.")
    if not np.issubdtype(pointers.dtype, np.integer):
        raise StructuralLookupError(
            f"{lookup.pointer_array} must contain integer offsets.")
    if not np.issubdtype(indices.dtype, np.integer):
        raise StructuralLookupError(
            f"{lookup.index_array} must contain integer coordinates.")


def materialize_structural_lookups(plan, argument_values, device=None):
    """Build every lookup table on the device.

    ``argument_values`` maps names to host arrays or device arrays; the result
    maps table names to device arrays (``DeviceArray``).  Violations of the
    structural properties raise :class:`StructuralLookupError`, as the
    reference's host loop does.
    """
    if not plan:
        return {}
    from lcd_amd import hip_runtime

    device = device or hip_runtime.default_device()
    values = {}
    for lookup in plan:
        try:
            pointers = argument_values[lookup.pointer_array]
            indices = argument_values[lookup.index_array]
        except KeyError as error:
            raise StructuralLookupError(
                f"Missing structural argument {error.args[0]!r}.") from error
        if isinstance(pointers, np.ndarray) or isinstance(pointers, (list, tuple)):
            validate_lookup_arrays(lookup, pointers, indices)
        try:
            values[lookup.name] = device.lookup_build(pointers, indices)
        except hip_runtime.HIPRuntimeError as error:
            if error.code in (hip_runtime.ERR_LOOKUP_POINTER,
                              hip_runtime.ERR_LOOKUP_ORDER):
                raise StructuralLookupError(str(error)) from error
            raise
    return values


__all__ = [
    "StructuralLookup", "StructuralLookupError",
    "create_structural_lookup_plan", "materialize_structural_lookups",
    "rewrite_structural_lookups", "structural_argument_names",
    "structural_lookup_names", "match_segment_search", "structure_aliases",
    "segmented_array_pairs",
]

"""DAG plans, the description of the inspector, and the GPU DAG builder.

Counterpart of compiler/dag_codegen.py of the reference.  The planner half is
:func:`create_dag_plan` (edge rules come from ``lcd_amd.dependence``);
:func:`direct_dependence` detects the push/pull protocols
(compiler/dag_codegen.py:1621-1664).  The emitter half is replaced: instead
of generating and exec-ing a Python ``extract_dag`` the plan is handed to
``lcdhip_dag_build``, which enumerates the same edges on the device.
:func:`generate_dag_source` still renders the enumeration as Python text, for
inspection and for tests that read the reference's generated inspector.
"""

import ast
from dataclasses import dataclass, field

import numpy as np

from lcd_amd.dependence import (
    GUARD_GREATER,
    GUARD_NONE,
    GUARD_NOT_EQUAL,
    LaterRule,
    NextRule,
    SegmentRule,
)

EXECUTION_MODES = frozenset({"sync_free", "wavefront"})
COUNTER_DEPENDENCE = "counter"
PUSH_DEPENDENCE = "push"
PULL_DEPENDENCE = "pull"
MAILBOX_DEPENDENCE = "mailbox"   # push edges delivered as per-entry messages
DEPENDENCE_PROTOCOLS = (COUNTER_DEPENDENCE, PUSH_DEPENDENCE, PULL_DEPENDENCE,
                        MAILBOX_DEPENDENCE)


class DAGCodegenError(Exception):
    """A dependence cannot be lowered to an efficient edge rule."""


EdgeRule = SegmentRule


@dataclass
class DAGPlan:
    arguments: list
    node_count: str            # source text of the task count, e.g. "n"
    edge_rules: list
    parallel_iterator: str
    node_lower: str = "0"


@dataclass(frozen=True)
class DirectDependence:
    """A task-level edge that the thread-mapped loop itself enumerates."""

    kind: str
    endpoint: ast.expr
    guard: ast.expr | None
    thread_loop: ast.For | None = field(default=None, compare=False)
    # the edges are enumerated by a sequential loop of the task (over
    # ``iterator``), not by the thread-mapped one: the task can wait for its
    # producers one by one, in the order it uses them
    sequential: bool = False
    iterator: str | None = None


def _normalize_execution_mode(execution_mode):
    execution_mode = execution_mode.replace("-", "_")
    if execution_mode not in EXECUTION_MODES:
        raise DAGCodegenError(
            f"Unknown execution mode {execution_mode!r}; expected one of "
            + ", ".join(sorted(EXECUTION_MODES)) + ".")
    return execution_mode


def create_dag_plan(ordering_dependences, node_data=None,
                    parallel_iterator="i", arguments=(), function_props=None,
                    node_count="n", node_lower="0"):
    """Collect the edge rules of the ordering dependences into a plan.

    ``ordering_dependences`` holds :class:`SegmentRule` objects (the output
    of ``analyze_dependences`` or hand-written rules).  Reduction dependences
    are rejected, as in the reference (test_dag_codegen.py:168-181).
    """
    rules = []
    for dependence in ordering_dependences:
        if getattr(dependence, "kind", None) == "reduction":
            raise DAGCodegenError(
                "Reduction dependences cannot be lowered to DAG edges.")
        if not isinstance(dependence, (SegmentRule, LaterRule, NextRule)):
            raise DAGCodegenError(
                "Edge rules must be SegmentRule, LaterRule or NextRule "
                "objects; got "
                f"{type(dependence).__name__}.")
        if dependence not in rules:
            rules.append(dependence)
    return DAGPlan(arguments=list(arguments), node_count=str(node_count),
                   edge_rules=rules, parallel_iterator=parallel_iterator,
                   node_lower=str(node_lower))


def _guard_source(rule):
    endpoint, owner = rule.endpoint_source(), rule.block_iterator
    source, destination = ((owner, endpoint) if rule.owner_is_source
                           else (endpoint, owner))
    if rule.guard == GUARD_GREATER:
        return f"{destination} > {source}"
    if rule.guard == GUARD_NOT_EQUAL:
        return f"{source} != {destination}"
    return None


def _range_source(rule):
    lower = f"{rule.pointer_array}[{rule.block_iterator}]"
    upper = f"{rule.pointer_array}[{rule.block_iterator} + 1]"
    if rule.lower_offset:
        lower += f" + {rule.lower_offset}" if rule.lower_offset > 0 else (
            f" - {-rule.lower_offset}")
    if rule.upper_offset:
        upper += f" + {rule.upper_offset}" if rule.upper_offset > 0 else (
            f" - {-rule.upper_offset}")
    return lower, upper


def generate_dag_source(plan, function_name="extract_dag",
                        validate_endpoints=False, execution_mode="sync_free",
                        edge_multiplicity=False):
    """Python text equivalent to what the device inspector enumerates."""
    mode = _normalize_execution_mode(execution_mode)
    n = plan.node_count
    lines = [f"def {function_name}({', '.join(plan.arguments)}):",
             f"    _dag_successors = [set() for _dag_node in range({n})]"]
    if edge_multiplicity:
        lines.append(f"    _dag_edge_count = [0 for _dag_node in range({n})]")
    for index, rule in enumerate(plan.edge_rules):
        it, inner = rule.block_iterator, rule.inner_iterator
        source, destination = f"_dag_source_{index}", f"_dag_destination_{index}"
        lines.append(f"    for {it} in range({plan.node_lower}, {n}):")
        if isinstance(rule, (LaterRule, NextRule)):
            upper = n if isinstance(rule, LaterRule) else (
                f"min({it} + {rule.lower_offset + 1}, {n})")
            lines.append(f"        for {inner} in range({it} + "
                         f"{rule.lower_offset}, {upper}):")
            lines.append(f"            {source} = {it}")
            lines.append(f"            {destination} = {inner}")
            lines.append(f"            _dag_successors[{source}]"
                         f".add({destination})")
            if edge_multiplicity:
                lines.append(f"            _dag_edge_count[{destination}] += 1")
            continue
        lower, upper = _range_source(rule)
        lines.append(f"        for {inner} in range({lower}, {upper}):")
        if rule.break_at_owner:
            lines.append(f"            if {rule.endpoint_source()} >= {it}:")
            lines.append("                break")
        endpoints = ((it, rule.endpoint_source()) if rule.owner_is_source
                     else (rule.endpoint_source(), it))
        lines.append(f"            {source} = {endpoints[0]}")
        lines.append(f"            {destination} = {endpoints[1]}")
        guards = []
        if validate_endpoints:
            guards += [f"0 <= {source} < {n}", f"0 <= {destination} < {n}"]
        guard = _guard_source(rule)
        if guard:
            guards.append(guard)
        body_indent = "            "
        if guards:
            lines.append(f"            if {' and '.join(guards)}:")
            body_indent += "    "
        lines.append(f"{body_indent}_dag_successors[{source}].add({destination})")
        if edge_multiplicity:
            lines.append(f"{body_indent}_dag_edge_count[{destination}] += 1")
    lines += [
        f"    dep_count = [0 for _dag_node in range({n})]",
        "    for _dag_neighbors in _dag_successors:",
        "        for _dag_destination in _dag_neighbors:",
        "            dep_count[_dag_destination] += 1",
    ]
    result = "dep_count"
    if mode == "wavefront":
        lines += [
            "    remaining_dep_count = list(dep_count)",
            "    wavefront_list = []",
            "    wavefront = [node for node, count in "
            "enumerate(remaining_dep_count) if count == 0]",
            "    while wavefront:",
            "        wavefront_list.append(wavefront)",
            "        new_wavefront = set()",
            "        for node in wavefront:",
            "            for successor in _dag_successors[node]:",
            "                remaining_dep_count[successor] -= 1",
            "                if remaining_dep_count[successor] == 0:",
            "                    new_wavefront.add(successor)",
            "        wavefront = sorted(new_wavefront)",
        ]
        result = "wavefront_list"
    returned = ("[sorted(_dag_neighbors) for _dag_neighbors in "
                f"_dag_successors], {result}")
    if edge_multiplicity:
        returned += ", _dag_edge_count"
    lines.append(f"    return ({returned})")
    return "\n".join(lines) + "\n"


def device_rules(plan, argument_values):
    """Bind the plan's rules to concrete structure arrays."""
    bound = []
    for rule in plan.edge_rules:
        if isinstance(rule, (LaterRule, NextRule)):
            bound.append(dict(relation=rule.relation,
                              lower_offset=rule.lower_offset))
            continue
        try:
            pointers = argument_values[rule.pointer_array]
            indices = argument_values[rule.index_array]
        except KeyError as error:
            raise DAGCodegenError(
                f"Missing structure argument {error.args[0]!r} for the DAG "
                "inspector.") from error
        if pointers is None or indices is None:
            raise DAGCodegenError(
                "The DAG inspector needs the structure arrays "
                f"{rule.pointer_array!r} and {rule.index_array!r}.")
        bound.append(dict(
            ptr=pointers, idx=indices, owner_is_source=rule.owner_is_source,
            lower_offset=rule.lower_offset, upper_offset=rule.upper_offset,
            guard=rule.guard, break_at_owner=rule.break_at_owner))
    return bound


def node_count_value(plan, argument_values):
    namespace = {"len": len}
    namespace.update(argument_values)
    count = eval(plan.node_count, {"__builtins__": {}}, namespace)
    lower = eval(plan.node_lower, {"__builtins__": {}}, namespace)
    if int(lower) != 0:
        raise DAGCodegenError(
            "The DAG inspector requires the block loop to start at 0.")
    return int(count)


def build_device_dag(plan, argument_values, device=None, levels=True,
                     force_kahn=False, incoming=False):
    """Run the on-device inspector for concrete inputs -> ``DeviceDag``."""
    from lcd_amd import hip_runtime

    device = device or hip_runtime.default_device()
    try:
        return device.dag_build(
            device_rules(plan, argument_values),
            node_count_value(plan, argument_values), levels=levels,
            force_kahn=force_kahn, incoming=incoming)
    except hip_runtime.HIPRuntimeError as error:
        if error.code == hip_runtime.ERR_DAG_BOUNDS:
            from lcd_amd.dag_preprocessing import DAGPreprocessingError
            raise DAGPreprocessingError(str(error)) from error
        raise


def compile_dag_builder(plan, function_name="extract_dag", globals_dict=None,
                        validate_endpoints=False, execution_mode="sync_free",
                        edge_multiplicity=False, device=None):
    """Return ``extract_dag(*args)`` with the reference's return convention
    (compiler/dag_codegen.py:1600-1618): ``(successor lists, dep_count |
    wavefront list[, edge_count])`` as Python lists, computed on the GPU."""
    mode = _normalize_execution_mode(execution_mode)

    def extract_dag(*args):
        values = dict(zip(plan.arguments, args))
        dag = build_device_dag(plan, values, device, levels=(mode == "wavefront"))
        scheduling = (dag.wavefront_list() if mode == "wavefront"
                      else dag.host("dep_count").tolist())
        result = (dag.successors(), scheduling)
        if edge_multiplicity:
            result += (dag.host("edge_count").tolist(),)
        return result

    extract_dag.__name__ = function_name
    extract_dag.plan = plan
    return extract_dag


def direct_dependence(plan, thread_iterator, validate_endpoints=False):
    """Push/pull detection: a single rule whose iterators are exactly the
    block and the thread iterator, without breaks."""
    if thread_iterator is None or len(plan.edge_rules) != 1:
        return None
    rule = plan.edge_rules[0]
    if not isinstance(rule, SegmentRule):
        return None
    if (rule.iterators[0] == plan.parallel_iterator
            and rule.iterators[1] != thread_iterator
            and not rule.owner_is_source and not validate_endpoints):
        # ILU0-CSR: `for k_ptr in <own segment>: k = idx[k_ptr]; if k >= i:
        # break; ...` -- the task reads producer k inside iteration k_ptr only
        endpoint = ast.parse(rule.endpoint_source(), mode="eval").body
        lower, upper = _range_source(rule)
        loop = ast.parse(
            f"for {rule.inner_iterator} in range({lower}, {upper}):\n    pass"
        ).body[0]
        guard_text = _guard_source(rule)
        return DirectDependence(
            kind=PULL_DEPENDENCE, endpoint=endpoint,
            guard=(ast.parse(guard_text, mode="eval").body
                   if guard_text else None),
            thread_loop=loop, sequential=True, iterator=rule.inner_iterator)
    if rule.iterators != [plan.parallel_iterator, thread_iterator]:
        return None
    if rule.break_at_owner:
        return None
    endpoint = ast.parse(rule.endpoint_source(), mode="eval").body
    guards = []
    if validate_endpoints:
        guards.append(f"0 <= {rule.endpoint_source()} < {plan.node_count}")
    guard_text = _guard_source(rule)
    if guard_text:
        guards.append(guard_text)
    guard = (ast.parse(" and ".join(guards), mode="eval").body
             if guards else None)
    lower, upper = _range_source(rule)
    loop = ast.parse(
        f"for {rule.inner_iterator} in range({lower}, {upper}):\n    pass"
    ).body[0]
    return DirectDependence(
        kind=PUSH_DEPENDENCE if rule.owner_is_source else PULL_DEPENDENCE,
        endpoint=endpoint, guard=guard, thread_loop=loop)


__all__ = [
    "COUNTER_DEPENDENCE", "PUSH_DEPENDENCE", "PULL_DEPENDENCE",
    "MAILBOX_DEPENDENCE",
    "DEPENDENCE_PROTOCOLS", "DAGCodegenError", "DAGPlan", "DirectDependence",
    "EdgeRule", "GUARD_GREATER", "GUARD_NONE", "GUARD_NOT_EQUAL", "LaterRule",
    "NextRule",
    "build_device_dag", "compile_dag_builder", "create_dag_plan",
    "direct_dependence", "generate_dag_source",
]

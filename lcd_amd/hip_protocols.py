"""Dependence protocols of the persistent executor (push, pull, mailbox and
its gathered form): their plans and the readiness code a task polls."""

import ast
import re
from copy import deepcopy

from lcd_amd.structural_lookups import structure_aliases
from lcd_amd.hip_emitter import (
    FLOAT,
    INT,
    PUSH_DEPENDENCE,
    _is_range_loop,
    _names_in,
)


# entries of a task record when level launches give a task to one lane
LEVEL_WIDE_ENTRIES = 4

class ProtocolMixin:
    """Methods of ``HIPLowerer`` (lcd_amd/hip_lowering.py)."""

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
        if ((self.execution_mode != "sync_free" and not self.level_pull)
                or self.block_task or self.chain_tasks
                or dependence.iterator is None):
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

    def _gather_poll_array(self):
        """What a consumer polls for a source outside its tile: the array
        itself, or its copy in queue order when sources are named by their
        place in the queue."""
        if self._tile is not None and self._tile.get("by_position"):
            return "_lcd_xq"
        return self._mailbox["array"]

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
        level = self._level_records
        if level is not None and records:
            # level order: the operands of the record's edges sit beside it
            loads = " ".join(
                f"{name} = {level['operands'][name]}"
                "[_task * LCD_TASK_LANES + _lane];"
                for name, _, _ in gather["operands"])
            if declare:
                lines.append(f"{pad}bool _g_queue = true; (void)_g_queue;")
        elif level is not None:
            # (further chunks name their sources by id)
            loads += " _g_queue = false;"
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
                + ("" if level is not None and "_g_pos" not in _names_in(
                    gather["value"]) else f"_g_pos = _lcd_rec_pos[{slot}]; ")
                + f"_g_src = _lcd_rec_src[{slot}]; {decode}"
                + " ".join(self._queue_load_lines) + " }")
            lines.append(f"{pad}{head} {{ {loads} }}")
            if self.single_chunk:
                # the first poll of a source outside the tile leaves with the
                # operand loads instead of one round trip later, in the poll
                # loop (128^3 grid: 0.354 -> 0.347 ms)
                # (with the flat queue every source is outside and mostly not
                # there yet at that time: 3 % slower, so tiles only)
                array = self._gather_poll_array()
                lines.append(f"{pad}double _g_early = lcd_empty();")
                if self._tile is not None:
                    lines.append(
                        f"{pad}{head[:-1]} && !_g_in) {{ _g_early = "
                        f"{self.poll_load}(&{array}[_g_src]); }}")
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

    def _fetch_pipeline(self, it, first_loads, first_zero, first, second_blocks,
                        task_of, bound, types):
        """Pieces of a fetch that runs two rounds deep.  ``first_loads`` are
        the loads addressed by the queue position alone (text over ``_t``),
        ``first`` the registers they fill; ``second_blocks`` are (condition,
        lines) pairs whose loads are named by the first ones.  Returns the
        declarations, the two request blocks (per register set and round
        expression) and the take-over lines."""
        import re
        kinds = self._kinds
        assigned = []
        for _, block in second_blocks:
            for line in block:
                for name in re.findall(
                        r"(?<![=!<>\w])([A-Za-z_]\w*)\s*=(?!=)", line):
                    if name not in assigned and name not in first:
                        assigned.append(name)
        second = assigned

        def ctype(name):
            if name in types:
                return types[name]
            if name == it:
                return "lcd_index_t"
            return ("double" if kinds.locals.get(name, INT) == FLOAT
                    else "lcd_index_t")

        pattern = re.compile(r"\b(" + "|".join(
            re.escape(name) for name in first + second + ["_task", "_pending"])
            + r")\b")

        def renamed(text, prefix):
            def swap(match):
                name = match.group(1)
                return {"_task": "_t", "_pending": "_v"}.get(
                    name, prefix + name)
            return pattern.sub(swap, text)

        def head(rounds):
            return (f"{{ const int _t = {task_of(rounds)}; const bool _v = "
                    f"_t < {bound}; (void)_v;")

        def request_first(prefix, rounds):
            return (f"{head(rounds)} "
                    + " ".join(f"{prefix}{name} = 0;" for name in first_zero)
                    + " if (_v) { "
                    + " ".join(renamed(line, prefix) for line in first_loads)
                    + " } }")

        def request_second(prefix, rounds):
            lines = [head(rounds)]
            for condition, block in second_blocks:
                lines.append(f"if (_v && ({renamed(condition, prefix)})) {{")
                lines += ["    " + renamed(line, prefix) for line in block]
                lines.append("}")
            lines.append("}")
            return lines

        declare = " ".join(
            [f"{ctype(name)} _a_{name} = 0;" for name in first]
            + [f"{ctype(name)} _b_{name} = 0;" for name in first + second])
        return {
            "declare": declare, "second": second,
            "request_first": request_first, "request_second": request_second,
            "take_first": " ".join(f"{name} = _b_{name};" for name in first),
            "take_second": " ".join(f"{name} = _b_{name};" for name in second),
            "shift": " ".join(f"_b_{name} = _a_{name};" for name in first),
        }

    def _prepared_reciprocal(self, taken):
        """The reciprocal of the task's divisor, prepared where a round takes
        over the node loads that were requested a round ago: the wavefront is
        about to wait for its producers, and the division that follows the
        wait -- on the chain between two levels -- shrinks to its last three
        operations and a range check (lcd_div_checked).  128^3 grid in box
        tiles: 0.238 -> 0.233 ms, bit for bit."""
        divisor = self._prepared_divisor
        if divisor is None or divisor not in taken:
            return []
        self._prepared_division_active = True
        return [f"_lcd_rcp = lcd_div_plain_divisor({divisor}) ? "
                f"lcd_div_prepare({divisor}) : lcd_empty();"]

    def _pipelined_fetch_lines(self, fetch, it):
        """Tiled executor with task records: the loads a round of tasks starts
        with, two rounds deep.  A wavefront's round began with two dependent
        trips to memory (the records of its tasks, then the operands the
        records name) during which it did nothing, and the tile advanced at
        the rate its wavefronts got through those trips, not at the rate of
        its LDS hand-offs.  Now a round takes over registers that were loaded
        while the rounds before it ran: the records of round r + 2 and the
        operands of round r + 1 are requested when round r starts.  (128^3
        grid: 0.347 -> 0.327 ms.)"""
        import re
        gather = self._mailbox["gather"]
        array = self._gather_poll_array()
        emitter = self._emitter
        split = next(index for index, line in enumerate(fetch)
                     if "for (int _round = 0" in line)
        queue_loads = list(self._queue_load_lines)
        queue_names = [re.match(r"\s*(\w+) = ", line).group(1)
                       for line in queue_loads]
        slot = "_task * LCD_TASK_LANES + _lane"
        first = [it, "_mb_next", "_mb_end", "_g_pos", "_g_src", *queue_names]
        operands = [name for name, _, _ in gather["operands"]]
        types = {"_mb_next": "int", "_mb_end": "int",
                 "_g_pos": "lcd_index_t", "_g_src": "lcd_index_t"}
        types.update({name: "lcd_index_t" if kind == INT else "double"
                      for name, _, kind in gather["operands"]})
        pipe = self._fetch_pipeline(
            it,
            [f"{it} = (lcd_index_t)task_nodes[_task];",
             "_mb_next = _lcd_rec_in[2 * _task];",
             "_mb_end = _lcd_rec_in[2 * _task + 1];",
             f"_g_pos = _lcd_rec_pos[{slot}];",
             f"_g_src = _lcd_rec_src[{slot}];", *queue_loads],
            [it, "_mb_next", "_mb_end"], first,
            [("_mb_next + _lane < _mb_end",
              [f"{name} = {emitter.expr(node)};"
               for name, node, _ in gather["operands"]]),
             (self._prefetch_guard, list(self._prefetch_lines))],
            lambda rounds: (
                f"(_lcd_tile_row0 + (({rounds}) * (LCD_TPB / 64) + "
                "(int)(threadIdx.x >> 6)) * _tasks_per_wave + "
                "(int)(threadIdx.x & 63) / LCD_TASK_LANES)"),
            "_lcd_tile_row0 + _lcd_tile_rows", types)
        tile_part, round_part = fetch[:split], fetch[split:]
        pad = "        "
        lines = list(tile_part)
        lines += ["    " + pipe["declare"],
                  "    " + pipe["request_first"]("_b_", "0"),
                  "    " + pipe["request_first"]("_a_", "1"),
                  *["    " + line for line in pipe["request_second"]("_b_", "0")]]
        lines += round_part
        lines += [
            f"{pad}{it} = 0;",
            f"{pad}int _mb_next = 0, _mb_end = 0;",
            f"{pad}lcd_index_t _g_pos = 0, _g_src = 0;",
            f"{pad}double _mb_value = lcd_empty();",
            *[f"{pad}{types[name]} {name} = 0;" for name in operands],
            f"{pad}unsigned _g_off = 0; bool _g_in = false;",
            # this round takes over what was loaded while the others ran
            f"{pad}if (_pending) {{ {pipe['take_first']} "
            "_g_off = (unsigned)(_g_src - _lcd_tile_row0); "
            "_g_in = _g_off < (unsigned)_lcd_tile_rows; }",
            f"{pad}{pipe['take_second']}",
            *[pad + line for line in self._prepared_reciprocal(pipe["second"])],
            f"{pad}{pipe['shift']}",
            *[pad + line for line in pipe["request_second"]("_b_", "_round + 1")],
            pad + pipe["request_first"]("_a_", "_round + 2"),
            f"{pad}double _g_early = lcd_empty();",
            f"{pad}if (_pending && _mb_next + _lane < _mb_end && !_g_in) "
            f"{{ _g_early = {self.poll_load}(&{array}[_g_src]); }}",
            f"{pad}const int _mb_have = (_mb_end - _mb_next) < "
            "LCD_TASK_LANES ? (_mb_end - _mb_next) : LCD_TASK_LANES;",
            f"{pad}bool _need = _pending && _lane < _mb_have;",
            f"{pad}const bool _fits = (_mb_end - _mb_next) <= LCD_TASK_LANES;",
        ]
        return lines

    def _pipelined_queue_fetch_lines(self, it):
        """The same two-round fetch for the flat level-ordered queue of the
        pull protocols: the task id and the structure loads addressed by the
        queue position for round r + 2, the node loads they name for round
        r + 1.  Tasks are dealt out round-robin (no shared counter), so a
        wavefront knows its later tasks.  (Power-law factor: 0.722 -> 0.69
        ms.)"""
        import re
        queue_loads = list(self._queue_load_lines)
        queue_names = [re.match(r"\s*(\w+) = ", line).group(1)
                       for line in queue_loads]
        first = [it, *queue_names]
        pipe = self._fetch_pipeline(
            it, [f"{it} = (lcd_index_t)task_nodes[_task];", *queue_loads],
            [it], first,
            [(self._prefetch_guard, list(self._prefetch_lines))],
            lambda rounds: (
                f"((({rounds}) * (int)(gridDim.x * (LCD_TPB / 64)) + "
                "(int)(blockIdx.x * (LCD_TPB / 64) + (threadIdx.x >> 6))) * "
                "_tasks_per_wave + (int)(threadIdx.x & 63) / LCD_TASK_LANES)"),
            "_task_count", {})
        pad = "        "
        return [
            "    int _round = 0;",
            "    " + pipe["declare"],
            "    " + pipe["request_first"]("_b_", "0"),
            "    " + pipe["request_first"]("_a_", "1"),
            *["    " + line for line in pipe["request_second"]("_b_", "0")],
            "    while (true) {",
            f"{pad}const int _base = (_round * (int)(gridDim.x * (LCD_TPB / 64)) + "
            "(int)(blockIdx.x * (LCD_TPB / 64) + (threadIdx.x >> 6))) * "
            "_tasks_per_wave;",
            f"{pad}++_round;",
            f"{pad}if (_base >= _task_count) return;",
            f"{pad}const int _task = _base + (int)(threadIdx.x & 63) / "
            "LCD_TASK_LANES;",
            f"{pad}bool _pending = _task < _task_count;",
            f"{pad}{it} = 0;",
            f"{pad}if (_pending) {{ {pipe['take_first']} }}",
            f"{pad}{pipe['take_second']}",
            # (no reciprocal prepared here: on the power-law factor it costs
            # more wavefront time than the shorter division gives back, 0.666
            # against 0.659 ms)
            f"{pad}{pipe['shift']}",
            *[pad + line for line in pipe["request_second"]("_b_", "_round")],
            pad + pipe["request_first"]("_a_", "_round + 1"),
        ]

    def _gather_ready_lines(self, indent):
        """Readiness for the gathered mailbox: lane ``l`` polls the final
        value of the producer of incoming edge ``next + l`` until it is there
        and keeps the product; once the lanes of a chunk all hold theirs, the
        products are added in (source, position) order -- the order of the
        sequential loop -- by broadcasting them lane by lane."""
        pad = "    " * indent
        own = self._mailbox["register"]
        gather = self._mailbox["gather"]
        array = self._gather_poll_array()
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
        if self._level_records is not None:
            # the record names a source by its place in the level order: the
            # value is read from the copy of the array in that order, which
            # the launch of the source's level wrote contiguously
            load = (f"(_g_queue ? _lcd_xq[_g_src] : {load})"
                    if not self.single_chunk else "_lcd_xq[_g_src]")
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
        elif self.task_lanes in (8, 16):
            # the group's first lane takes the products one by one (DPP row
            # shifts) and adds them in order; its total goes to the group
            ordered = [
                f"{pad}        {{ const double _mb_in = lcd_row_take<{k}>(_mb_value); "
                f"if ({k} < _mb_have) {own} = {own} + _mb_in; }}"
                for k in range(self.task_lanes)]
            ordered.append(
                f"{pad}        {own} = lcd_group_first<LCD_TASK_LANES>({own});")
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
                "{ const double _g_raw = lcd_is_empty(_g_early) ? "
                + ("_lcd_xq[_g_src]" if self._level_records is not None
                   else f"{self.poll_load}(&{array}[_g_src])")
                + " : _g_early; "
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

    def _level_records_plan(self, body):
        """Level launches over operands in level order.  A launch then reads
        contiguous memory only: the record of a task (its first incoming
        edges), the operands of those edges, the task's node values, and the
        values of its sources from a copy of the array in level order that
        the tasks write beside the array itself.  The copies are filled by
        two staging kernels that share the kernel's signature: one for what
        comes from the arrays the edge operands read (the matrix; run again
        when their contents change), one for the rest of the node values
        (the right-hand side; run in front of every call).  Returns the plan,
        or None when the task does not fit: a host loop around the launches,
        an operand or a product that names its source by id, a store to the
        array at another place than the task's own."""
        gather, kinds = self._mailbox["gather"], self._kinds
        array = self._mailbox["array"]
        if self.host_loops or self.chain_tasks:
            return None
        if "_g_src" in _names_in(gather["value"]):
            return None
        operands = {}
        static_arrays = []
        for index, (name, node, kind) in enumerate(gather["operands"]):
            if "_g_src" in _names_in(node.slice):
                return None
            operands[name] = f"_lcd_lr_{index}"
            kinds.arrays[operands[name]] = kind
            for sub in ast.walk(node):
                if (isinstance(sub, ast.Subscript)
                        and isinstance(sub.value, ast.Name)
                        and kinds.arrays.get(sub.value.id) == FLOAT
                        and sub.value.id not in static_arrays):
                    static_arrays.append(sub.value.id)
        for statement in body:
            for node in ast.walk(statement):
                targets = (node.targets if isinstance(node, ast.Assign) else
                           [node.target] if isinstance(node, ast.AugAssign)
                           else [])
                for target in targets:
                    if (isinstance(target, ast.Subscript)
                            and isinstance(target.value, ast.Name)
                            and target.value.id == array
                            and not (isinstance(target.slice, ast.Name)
                                     and target.slice.id == self.loop_iterator)):
                        if node is not self._mailbox["sites"][0]:
                            return None
        kinds.arrays["_lcd_xq"] = FLOAT
        function_name = self._sweep_function_name
        wide = self.task_lanes == 1
        if wide:
            # a task per lane: its record has LEVEL_WIDE_ENTRIES entries,
            # fetched with vector loads (`_level_wide_fetch_lines`)
            self.record_lanes = LEVEL_WIDE_ENTRIES
        return {"operands": operands, "values": [], "order": [], "wide": wide,
                "static_arrays": static_arrays, "dynamic": False,
                "kernels": (function_name + "_hip_level_static",
                            function_name + "_hip_level_dynamic")}

    def _level_wide_fetch_lines(self, indent):
        """Level records with a task per lane: the record's sources and the
        operands of its edges come in with one vector load per array (the
        addresses depend on the task's place in the level order alone), the
        node values beside them."""
        pad = "    " * indent
        level, gather = self._level_records, self._mailbox["gather"]
        lines = [
            f"{pad}const int _mb_begin = _lcd_rec_in[2 * _task], "
            "_mb_end = _lcd_rec_in[2 * _task + 1];",
            f"{pad}const int _mb_have = (_mb_end - _mb_begin) < "
            "LCD_RECORD_LANES ? (_mb_end - _mb_begin) : LCD_RECORD_LANES;",
            f"{pad}const int4 _g_s = ((const int4*)_lcd_rec_src)[_task];",
            f"{pad}const lcd_index_t _g_srcs[4] = {{_g_s.x, _g_s.y, _g_s.z, "
            "_g_s.w};"]
        for name, _, kind in gather["operands"]:
            vector = "int4" if kind == INT else "double4"
            scalar = "lcd_index_t" if kind == INT else "double"
            staged = level["operands"][name]
            lines += [
                f"{pad}const {vector} {name}_v = "
                f"((const {vector}*){staged})[_task];",
                f"{pad}const {scalar} {name}_w[4] = {{{name}_v.x, {name}_v.y, "
                f"{name}_v.z, {name}_v.w}};"]
        return lines

    def _level_wide_sum_lines(self, indent):
        """... and the task's sum: the sources' values from the copy of the
        array in level order, all loads in flight together, the products
        added in the order of the record (the order of the sequential loop);
        entries beyond the record are read by id, one by one."""
        pad = "    " * indent
        gather, emitter = self._mailbox["gather"], self._emitter
        own = self._mailbox["register"]
        array = self._mailbox["array"]

        sign = "-" if gather["negate"] else ""
        lines = [f"{pad}double _g_values[4] = {{0.0, 0.0, 0.0, 0.0}};",
                 f"{pad}#pragma unroll",
                 f"{pad}for (int _e = 0; _e < LCD_RECORD_LANES; ++_e) "
                 "if (_e < _mb_have) _g_values[_e] = _lcd_xq[_g_srcs[_e]];"]
        for entry in range(LEVEL_WIDE_ENTRIES):
            lines.append(
                f"{pad}if ({entry} < _mb_have) {own} = {own} + "
                f"{sign}({self._wide_product_text(entry)});")
        if not self.single_chunk:
            operands = " ".join(
                f"const {'lcd_index_t' if kind == INT else 'double'} {name} = "
                f"{emitter.expr(node)};" for name, node, kind in gather["operands"])
            lines += [
                f"{pad}for (int _e = _mb_begin + LCD_RECORD_LANES; _e < _mb_end; "
                "++_e) {",
                f"{pad}    const lcd_index_t _g_pos = _lcd_in_pos[_e]; (void)_g_pos;",
                f"{pad}    const lcd_index_t _g_src = _lcd_in_src[_e];",
                f"{pad}    {operands}",
                f"{pad}    const double _g_value = {array}[_g_src];",
                f"{pad}    {own} = {own} + {sign}({emitter.expr(gather['value'])});",
                f"{pad}}}"]
        return lines

    def _wide_product_text(self, entry):
        """The product of one record entry, over the registers the wide
        fetch filled."""
        gather, emitter = self._mailbox["gather"], self._emitter
        text = emitter.expr(gather["value"])
        for name, _, _ in gather["operands"]:
            text = re.sub(rf"\b{re.escape(name)}\b", f"{name}_w[{entry}]", text)
        return re.sub(r"\b_g_value\b", f"_g_values[{entry}]", text)

    def _level_value_load(self, name, node, text):
        """A node value ``R[e]`` of a read-only float array in level order:
        ``_lcd_lv_k[_task]``, or None when it stays a load by id."""
        level = self._level_records
        if level is None or self._kinds.arrays.get(node.value.id) != FLOAT:
            return None
        if any(isinstance(sub, ast.Name) and sub.id.startswith("_nl_")
               and self._kinds.locals.get(sub.id) == FLOAT
               for sub in ast.walk(node.slice)):
            return None
        staged = f"_lcd_lv_{len(level['values'])}"
        static = node.value.id in level["static_arrays"]
        level["values"].append((name, staged, text, static))
        level["dynamic"] = level["dynamic"] or not static
        self._kinds.arrays[staged] = FLOAT
        return staged

    def _level_stage_kernels(self, function_name, signature, declarations,
                             guard):
        """The two staging kernels of the level records (same signature as
        the level kernel; ``band_start`` = 0 and ``band_end`` = the number of
        tasks).  Static: a thread per slot of the records; dynamic: a thread
        per task."""
        level, gather = self._level_records, self._mailbox["gather"]
        emitter, it = self._emitter, self.loop_iterator
        static_name, dynamic_name = level["kernels"]

        def head(name, per_task):
            lines = ["", 'extern "C" __global__ void __launch_bounds__(256)',
                     f"{name}(", f"        {signature})", "{",
                     *declarations,
                     f"    lcd_index_t {it} = 0;",
                     "    const long long _slot = (long long)blockIdx.x * "
                     "blockDim.x + threadIdx.x;"]
            if per_task:
                lines += ["    const long long _task = (long long)band_start "
                          "+ _slot;",
                          "    const int _lane = 0; (void)_lane;"]
            else:
                lines += ["    const long long _task = (long long)band_start "
                          "+ _slot / LCD_RECORD_LANES;",
                          "    const int _lane = (int)(_slot % LCD_RECORD_LANES);"]
            lines += ["    if (_task >= band_end) return;",
                      f"    {it} = task_nodes[_task];"]
            return lines

        def values(static):
            lines = []
            for kind, line, is_static in level["order"]:
                if kind == "value":
                    if is_static == static:
                        lines.append(f"        {line}")
                else:
                    lines.append(f"        {line}")
            return lines

        loads = [f"            {level['operands'][name]}[_slot] = "
                 f"{emitter.expr(node)};"
                 for name, node, _ in gather["operands"]]
        clears = [f"            {level['operands'][name]}[_slot] = 0;"
                  for name, _, _ in gather["operands"]]
        static = head(static_name, False) + [
            f"    if ({guard}) {{",
            "        if (_lane == 0) {",
            *["    " + line for line in values(True)],
            "        }",
            "        const int _mb_next = _lcd_rec_in[2 * _task], "
            "_mb_end = _lcd_rec_in[2 * _task + 1];",
            "        if (_mb_next + _lane < _mb_end) {",
            "            const lcd_index_t _g_pos = _lcd_rec_pos[_slot]; "
            "(void)_g_pos;",
            *loads,
            "        } else {",
            *clears,
            "        }",
            "    }",
            "}", ""]
        dynamic = head(dynamic_name, True) + [
            f"    if ({guard}) {{",
            *values(False),
            "    }",
            "}", ""]
        return "\n".join(static + dynamic)

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

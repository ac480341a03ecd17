"""Pull protocol on a sequential loop of the task (ILU0's pivot loop): the
resumable loop with `done` flags and the pipelined loop over published
values."""

import ast
from copy import deepcopy

from lcd_amd.hip_emitter import (
    FLOAT,
    INT,
    STATUS_ARGUMENT,
    VALUE_WAIT_BEGIN,
    VALUE_WAIT_END,
)


# Level launches: how many producers of a task are read "flat" -- every table
# entry of all of them asked for at once, then every value, then the
# arithmetic producer by producer -- before the producer loop takes the rest.
LEVEL_FLAT_PRODUCERS = 4


class SequentialPullMixin:
    """Methods of ``HIPLowerer`` (lcd_amd/hip_lowering.py)."""

    def _sequential_pull_lines(self, node, emitter, hooks, lower, upper):
        """The task's loop over its producers, resumable: every iteration
        first checks that its producer has published ``done`` and otherwise
        leaves the loop with the position kept; the lines between the two
        markers are re-entered by the executor's poll loop.  The task works
        on the producers that are finished while it waits for the others.
        With published values there is no flag to wait for (the reads of the
        producer's entries poll) and the loop runs through in one go, in its
        pipelined form where the body allows."""
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
                        and call.func.id in ("_lcd_sorted_find",
                                             "_lcd_pair_at"))
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
        # With the own segment in registers and the searches in tables the
        # loop runs to a bound the wavefront counts when it takes the task
        # (`_counted_producer_plan`): no load of the producer's id and no
        # test on it per iteration.
        counted = None
        segment = self._segment or {}
        if (leave is not None and leave == 1 and len(before) == 1
                and segment.get("registers") and segment.get("counted")
                and self._structure_tables
                and name == self._sequential_pull["iterator"]
                and segment["counted"]["producer"] == before[0].targets[0].id):
            counted = segment["counted"]
            bound = ast.Name(id="_lcd_low_end", ctx=ast.Load())
            self._kinds.locals["_lcd_low_end"] = INT
            self._kinds.locals["_lcd_low_at"] = INT
            self._own_registers += ["_lcd_low_end", "_lcd_low_at"]

            class AtLane(ast.NodeTransformer):
                def visit_Name(self, sub):
                    if sub.id == counted["producer"]:
                        return ast.copy_location(ast.Subscript(
                            value=ast.Name(id=counted["index"], ctx=ast.Load()),
                            slice=ast.Name(id="_lcd_low_at", ctx=ast.Load()),
                            ctx=ast.Load()), sub)
                    return sub

            leaves = emitter.expr(ast.fix_missing_locations(
                AtLane().visit(deepcopy(leading[leave].test))))
            count_lines = [
                "{",
                "    _lcd_low_at = _lcd_seg_base + _lane;",
                f"    const bool _lcd_low_stop = _lane < _lcd_seg_own && "
                f"_lcd_low_at >= {lower} && _lcd_low_at < "
                f"{emitter.expr(upper)} && {leaves};",
                "    const unsigned long long _lcd_low_mask = "
                "__ballot(_lcd_low_stop);",
                "    _lcd_low_end = _lcd_low_mask ? _lcd_seg_base + "
                "(lcd_index_t)__ffsll((long long)_lcd_low_mask) - 1 : "
                f"{emitter.expr(upper)};",
                "}",
            ]
            if not counted["used"]:
                before = []
            upper, leave = bound, None
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
        table_names = {entry[1] for entry in self._structure_tables}
        index_arrays = {entry[3] for entry in self._structure_tables}

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
            if leave is not None and not speculative:
                body = [ast.If(test=ast.UnaryOp(
                    op=ast.Not(), operand=Shift().visit(
                        deepcopy(leading[leave].test))), body=body, orelse=[])]
            return ast.fix_missing_locations(ast.If(
                test=ast.Compare(left=deepcopy(position), ops=[ast.Lt()],
                                 comparators=[deepcopy(upper)]),
                body=shifted + body, orelse=[]))

        # With the structure searches in tables every address the located
        # statements read depends on positions of the task's own segment
        # (inside it whenever the position is): they need not wait for the
        # test that leaves the loop, which depends on a load itself.
        speculative = bool(self._structure_tables) and not any(
            isinstance(sub, ast.Call) and isinstance(sub.func, ast.Name)
            and sub.func.id == "_lcd_sorted_find"
            for statement in structure for sub in ast.walk(statement)) and all(
                isinstance(sub.value, ast.Name)
                and (sub.value.id in table_names
                     or sub.value.id in index_arrays)
                for statement in structure for sub in ast.walk(statement)
                if isinstance(sub, ast.Subscript))
        rest = list(node.body[split:])
        leading_loads = self._split_leading_loads(rest)
        first_loads = list(fetched) + leading_loads
        take_over = [ast.fix_missing_locations(ast.Assign(
            targets=[ast.Name(id=local, ctx=ast.Store())],
            value=ast.Name(id=f"_nx_{local}", ctx=ast.Load())))
            for local in names]
        lines = [f"{name} = {lower};"]
        flat = None
        if (counted is not None and speculative and leave is None
                and self._published.get("plain")):
            flat = self._flat_producers(
                name, node.iter.args[1], before + structure, names,
                first_loads, take_over, rest, emitter, hooks)
        if flat is not None:
            lines += flat[0] + count_lines + flat[1]
        else:
            lines += count_lines if counted else []
        lines += self._emit_guarded(ahead(0), emitter, 0, hooks)
        lines += [VALUE_WAIT_BEGIN, "_lcd_blocked = false;",
                  f"for (; {name} < {emitter.expr(upper)}; ++{name}) {{"]
        for child in take_over + ([] if leave is None else [leading[leave]]):
            lines += self._emit_guarded(child, emitter, 1, hooks)
        # the next producer's row is searched while this one's values are on
        # their way.  (Sending the next one's first loads too, once these
        # values are here, was slower: 8.2 against 7.2 ms on the 9-point
        # grid -- most come back empty, and every extra coherent load slows
        # the hand-offs.)
        for child in first_loads + [ahead(1)]:
            lines += self._emit_guarded(child, emitter, 1, hooks)
        # the statements that wait for the leading loads (the producer's
        # diagonal) come first in the rest; behind the last of them the
        # lanes' own first loads get their second attempt
        again = (self._second_attempts(fetched, emitter)
                 if leading_loads and not self._published.get("plain")
                 else [])
        for position, child in enumerate(rest):
            lines += self._emit_guarded(child, emitter, 1, hooks)
            if position == len(leading_loads) - 1:
                for guard, register, load in again:
                    lines.append(f"    if (({guard}) && lcd_is_empty({register})) "
                                 f"{register} = {load};")
        lines += ["}", VALUE_WAIT_END]
        return lines

    def _flat_producers(self, name, row_end, located, names, first_loads,
                        take_over, rest, emitter, hooks):
        """Level launches (every producer ran in an earlier launch, nothing
        is polled): the first ``LEVEL_FLAT_PRODUCERS`` producers of a task
        without the chain of dependent trips the producer loop makes of
        them.  What the located statements read from the inspector's tables
        is asked for at once for all of them, through loads that no guard
        encloses (an entry that is not there -- the producer beyond the
        loop's end, the lane without an entry -- reads entry 0 instead: a
        guarded load keeps its wait inside the guard, and the trips come
        back); then the values they point at, the same way; then the
        iterations themselves, which find everything in registers.  Returns
        (lines in front of the count of the loop's bound, lines behind it),
        or None where a statement has a shape this does not know (the
        producer loop then does all the work, as it does for the producers
        after these)."""
        flat = LEVEL_FLAT_PRODUCERS
        kinds = self._kinds
        tables = ({entry[1] for entry in self._structure_tables}
                  | {entry[3] for entry in self._structure_tables})
        loaded = []
        for statement in first_loads:
            for sub in ast.walk(statement):
                if (isinstance(sub, ast.Name) and isinstance(sub.ctx, ast.Store)
                        and sub.id not in loaded):
                    loaded.append(sub.id)

        def pure(node):
            for sub in ast.walk(node):
                if isinstance(sub, ast.Subscript):
                    return False
                if isinstance(sub, ast.Call) and not (
                        isinstance(sub.func, ast.Name)
                        and sub.func.id == "_lcd_rseg_first"):
                    return False
            return True

        def renamed(node, q):
            prefix = f"_f{q}_"

            class Rename(ast.NodeTransformer):
                def visit_Name(self, sub):
                    if sub.id in names or sub.id in loaded:
                        return ast.copy_location(
                            ast.Name(id=prefix + sub.id, ctx=sub.ctx), sub)
                    if sub.id == name and q:
                        return ast.copy_location(ast.BinOp(
                            left=ast.Name(id=name, ctx=ast.Load()),
                            op=ast.Add(), right=ast.Constant(value=q)), sub)
                    return sub

            return ast.fix_missing_locations(Rename().visit(deepcopy(node)))

        def both(guard, test):
            return test if guard is None else f"({guard}) && ({test})"

        ask, settle, values, work = [], [], [], []
        for q in range(flat):
            here = (f"({name} + {q}) < {emitter.expr(row_end)}" if q
                    else f"{name} < {emitter.expr(row_end)}")
            on = (f"({name} + {q}) < _lcd_low_end" if q
                  else f"{name} < _lcd_low_end")

            def locate(statement, guard):
                if isinstance(statement, ast.If) and not statement.orelse:
                    if not pure(statement.test):
                        return False
                    test = emitter.expr(renamed(statement.test, q))
                    return all(locate(child, both(guard, test))
                               for child in statement.body)
                if not (isinstance(statement, ast.Assign)
                        and len(statement.targets) == 1
                        and isinstance(statement.targets[0], ast.Name)):
                    return False
                target = f"_f{q}_{statement.targets[0].id}"
                value = statement.value
                if pure(value):
                    text = f"{target} = {emitter.expr(renamed(value, q))};"
                    ask.append(text if guard is None
                               else f"if ({guard}) {text}")
                    return True
                if (isinstance(value, ast.Subscript)
                        and isinstance(value.value, ast.Name)
                        and value.value.id in tables and pure(value.slice)):
                    index = emitter.expr(renamed(value.slice, q))
                    ask.append(f"{target} = {value.value.id}"
                               f"[({both(guard, here)}) ? {index} : 0];")
                    return True
                if (isinstance(value, ast.Call)
                        and isinstance(value.func, ast.Name)
                        and value.func.id == "_lcd_pair_at"
                        and len(value.args) == 2
                        and all(pure(arg) for arg in value.args)):
                    row, at = (emitter.expr(renamed(arg, q))
                               for arg in value.args)
                    where = both(guard, here)
                    for part in ("_o", "_s"):
                        kinds.locals[target + part] = INT
                        self._own_registers.append(target + part)
                    ask.append(
                        f"{target}_o = _lcd_pair[({where}) ? _lcd_pair_row + "
                        f"(({row}) - _lcd_seg_base) * _lcd_seg_own + "
                        f"(({at}) - _lcd_seg_base) : 0];")
                    ask.append(f"{target}_s = _lcd_pair_start"
                               f"[({where}) ? {row} : 0];")
                    settle.append(
                        f"{target} = ({both(guard, on)}) ? "
                        f"lcd_pair_pos({target}_o, {target}_s) : -1;")
                    return True
                return False

            if not all(locate(statement, None) for statement in located):
                return None
            for statement in first_loads:
                test, body = None, [statement]
                if isinstance(statement, ast.If) and not statement.orelse:
                    if not pure(statement.test):
                        return None
                    test = emitter.expr(renamed(statement.test, q))
                    body = statement.body
                for child in body:
                    if not (isinstance(child, ast.Assign)
                            and len(child.targets) == 1
                            and isinstance(child.targets[0], ast.Name)
                            and isinstance(child.value, ast.Call)
                            and isinstance(child.value.func, ast.Name)
                            and child.value.func.id == "_lcd_raw"
                            and len(child.value.args) == 1
                            and isinstance(child.value.args[0], ast.Subscript)
                            and isinstance(child.value.args[0].value, ast.Name)
                            and pure(child.value.args[0].slice)):
                        return None
                    source = child.value.args[0]
                    index = emitter.expr(renamed(source.slice, q))
                    values.append(
                        f"_f{q}_{child.targets[0].id} = {source.value.id}"
                        f"[({both(test, on)}) ? {index} : 0];")
            work.append(f"if ({name} < _lcd_low_end) {{")
            for local in names + loaded:
                work.append(f"    {local} = _f{q}_{local};")
            for child in rest:
                work += self._emit_guarded(child, emitter, 1, hooks)
            work += [f"    ++{name};", "}"]
        for q in range(flat):
            for local in names + loaded:
                kinds.locals[f"_f{q}_{local}"] = kinds.locals.get(local, INT)
                self._own_registers.append(f"_f{q}_{local}")
        return ask, settle + values + work

    def _second_attempts(self, first_loads, emitter):
        """Second attempt of an iteration's first loads, once, behind the
        wait for the first of them.  A producer stores its entries with one
        instruction, so a diagonal that was not there yet means the lane's
        other entry was not either; its second attempt used to start where
        the value is used, behind the division, one more round trip on the
        chain between two levels.  Now it leaves as soon as the diagonal is
        in and arrives while the division runs.  (Polling all of them in one
        loop until the last has arrived was slower, 4.92 against 4.20 ms on
        the 9-point grid: every additional coherent load per poll slows
        everybody's hand-offs.)"""
        waits = []
        for statement in first_loads:
            guard = "1"
            if isinstance(statement, ast.If):
                guard = emitter.expr(statement.test)
                statement = statement.body[0]
            if not (isinstance(statement, ast.Assign)
                    and isinstance(statement.targets[0], ast.Name)
                    and isinstance(statement.value, ast.Call)
                    and isinstance(statement.value.func, ast.Name)
                    and statement.value.func.id == "_lcd_raw"):
                return []
            waits.append((guard, statement.targets[0].id,
                          emitter.expr(statement.value)))
        return waits

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
                         and call.func.id in ("_lcd_sorted_find",
                                              "_lcd_pair_at"))
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
        registers = (self._segment is not None
                     and self._segment.get("registers")
                     and iterator in self._segment["owned"])
        if registers:
            # lane l works on entry l of the segment, once
            first = ast.Assign(
                targets=[ast.Name(id="_sp_first", ctx=ast.Store())],
                value=ast.Call(
                    func=ast.Name(id="_lcd_rseg_first", ctx=ast.Load()),
                    args=[deepcopy(lower)], keywords=[]))
        else:
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
        if registers:
            # the lane's only iteration is the one located ahead of the wait
            pick_up = ast.If(test=ast.Constant(value=True),
                             body=pick_up.body, orelse=[])
        rest = mapped.body[len(structural):]
        fetched = self._fetch_behind_wait(rest, iterator, names, renamed, upper,
                                          single_trip=registers)
        mapped.body = [pick_up] + rest
        early = [first, ahead]
        for statement in early + fetched + [pick_up]:
            ast.fix_missing_locations(statement)
        return early, fetched

    def _fetch_behind_wait(self, rest, iterator, names, renamed, upper,
                           single_trip=False):
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
                if single_trip:
                    return ast.copy_location(held, node)
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

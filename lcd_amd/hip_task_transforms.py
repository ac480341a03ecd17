"""Rewrites of a task body ahead of emission: privatised scalars, staged
own segments and tiles, forwarded stores, promoted own elements, hoisted and
queue-ordered node loads."""

import ast
from copy import deepcopy

from lcd_amd.dependence import _split_offset
from lcd_amd.hip_emitter import (
    FLOAT,
    HIPLoweringError,
    INT,
    STATUS_ARGUMENT,
    _is_range_loop,
    _names_in,
    _stored_names,
)


class TaskTransformMixin:
    """Methods of ``HIPLowerer`` (lcd_amd/hip_lowering.py)."""

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
        if (self._published is not None and self._segment is not None
                and self.execution_mode == "sync_free"
                and len(target_loop.iter.args) == 1):
            # published pull (ILU0): the tile's slice of the publication
            # buffer, positions P[row0] .. P[row0 + rows), has a copy in LDS;
            # a tile whose slice is longer than the copy runs without it
            positions = self.tile_positions or min(16 * rows, 9216)
            if not isinstance(positions, int) or not 0 < positions <= 19456:
                raise HIPLoweringError(
                    "tile_positions must be a positive integer of at most "
                    "19456 (152 KB of LDS).")
            # the staged rows share the workgroup's LDS (160 KB) with the copy
            groups = max(1, self.threads_per_block // self.task_lanes)
            room = (160 * 1024 - 1024 - 8 * positions) // (8 * groups)
            if room < 8:
                raise HIPLoweringError(
                    f"tile_positions={positions} leaves no LDS for the rows "
                    f"of {groups} tasks per workgroup.")
            self._segment["capacity"] = min(self._segment["capacity"], room)
            return {"array": self._published["array"], "rows": rows,
                    "published": True, "positions": positions,
                    "pointer": self._segment["pointer"]}
        array = None
        if self._value_pull is not None:
            array = self._value_pull["array"]
        elif self._mailbox is not None and self._mailbox["gather"] is not None:
            array = self._mailbox["array"]
        if (array is None or self.execution_mode != "sync_free"
                or self.block_task or len(target_loop.iter.args) != 1):
            return None      # the flat queue serves every other combination
        return {"array": array, "rows": rows}

    def _tile_by_position_plan(self):
        """Tiles that do not follow the ids (boxes of a grid): a tile is
        ``tile_rows`` consecutive places of the task queue, whatever ids sit
        there.  The task records then name a source by its place in the
        queue, the LDS slot of a source is its place minus the tile's first,
        and the value-as-flag copy that other tiles poll is a buffer in queue
        order (``_lcd_xq``); the array itself gets plain stores and needs no
        reset.  Needs the gathered mailbox with task records that hold every
        incoming edge, and products that do not use the producer's id."""
        tile, mailbox = self._tile, self._mailbox
        gather = mailbox["gather"] if mailbox is not None else None
        if (tile is None or tile.get("published") or gather is None
                or not gather.get("records") or not self.single_chunk):
            return
        names = set(_names_in(gather["value"]))
        for _, node, _ in gather["operands"]:
            names |= set(_names_in(node))
        if "_g_src" in names:
            return
        tile["by_position"] = True
        self._kinds.arrays["_lcd_xq"] = FLOAT

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
        plan = {"array": array, "pointer": next(iter(pointers)),
                "capacity": capacity, "owned": set(owned), "registers": False}
        if self.segment_registers and self.task_lanes == 64:
            # (decided once the protocol is known: `_segment_registers_plan`)
            plan["capacity"] = 64
        return plan

    def _segment_registers_plan(self, body):
        """Keeps the task's own segment in registers instead of LDS: lane l
        of the task's wavefront holds entry l.  For a caller that knows every
        segment has at most 64 entries (``segment_registers=True``), with one
        wavefront per task and published values; every store to the array
        must go through a loop variable that walks the segment.  The chain
        between two levels loses its LDS round trips (store -> fence -> load
        per update) and the distributed loop its second path: a lane visits
        one entry, the one it holds."""
        plan = self._segment
        if not (self.segment_registers and plan is not None
                and self._published is not None and self.task_lanes == 64
                and self._sequential_pull is not None
                and self.thread_unroll_factor == 1):
            return
        array, owned = plan["array"], plan["owned"]
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
                            and target.value.id == array
                            and not (isinstance(target.slice, ast.Name)
                                     and target.slice.id in owned)):
                        return
        plan["registers"] = True
        plan["capacity"] = 64

    def _pair_table_plan(self, body):
        """With the own segment in registers (every segment of the structure
        has at most 64 entries) the searches the task makes per producer are
        read from tables the inspector builds once per structure:

        * ``L[k]`` with ``k = IDX[p]``, ``p`` the position in the own segment
          the sequential producer loop is at and ``L`` a structural lookup
          table over (PTR, IDX): ``_lcd_at_<L>[p]`` (the table gathered
          through IDX);
        * ``find(IDX, PTR[k], PTR[k + 1], j)`` with ``j = IDX[q]``, ``q`` the
          distributed loop's position in the own segment:
          ``_lcd_pair_start[p] + _lcd_pair[_lcd_pair_base[i] + (p - PTR[i]) * len
          + (q - PTR[i])]`` (a table of byte offsets, -1 where there is none,
          and ``_lcd_pair_start[p] = PTR[IDX[p]]``).

        Every address then depends on the task's own positions alone: the
        chain producer id -> its segment bounds -> its entries (three
        dependent loads per producer) is gone.  The rewrite is in place;
        returns the tables the runtime has to provide."""
        plan, pull = self._segment, self._sequential_pull
        if not (self.pair_tables and plan is not None and plan.get("registers")
                and pull is not None and self.thread_loop_iterator is not None):
            return ()
        pointer, owned = plan["pointer"], plan["owned"]
        outer_name, inner_name = pull["iterator"], self.thread_loop_iterator
        if outer_name not in owned or inner_name not in owned:
            return ()
        outer = next((s for s in body if isinstance(s, ast.For)
                      and isinstance(s.target, ast.Name)
                      and s.target.id == outer_name), None)
        if outer is None:
            return ()
        inner = next((n for n in ast.walk(outer) if isinstance(n, ast.For)
                      and isinstance(n.target, ast.Name)
                      and n.target.id == inner_name), None)
        written = self._all_written
        lookups = {lookup.name: lookup for lookup in self.structural_lookups}

        def gathered(statements, position):
            """name -> IDX for the single assignments ``name = IDX[position]``
            of a loop body."""
            found, counts = {}, {}
            for node in ast.walk(ast.Module(body=list(statements),
                                            type_ignores=[])):
                if isinstance(node, ast.Name) and isinstance(node.ctx, ast.Store):
                    counts[node.id] = counts.get(node.id, 0) + 1
            for statement in statements:
                if (isinstance(statement, ast.Assign)
                        and len(statement.targets) == 1
                        and isinstance(statement.targets[0], ast.Name)
                        and isinstance(statement.value, ast.Subscript)
                        and isinstance(statement.value.value, ast.Name)
                        and statement.value.value.id not in written
                        and isinstance(statement.value.slice, ast.Name)
                        and statement.value.slice.id == position
                        and counts.get(statement.targets[0].id) == 1):
                    found[statement.targets[0].id] = statement.value.value.id
            return found

        producers = gathered(outer.body, outer_name)
        columns = gathered(inner.body, inner_name) if inner is not None else {}
        tables = []

        def table_for(kind, *key):
            for entry in tables:
                if entry[0] == kind and entry[2:] == key:
                    return entry[1]
            name = (f"_lcd_at_{key[0]}" if kind == "at" else
                    "_lcd_pair_start" if kind == "start" else "_lcd_pair")
            tables.append((kind, name, *key))
            return name

        class Rewrite(ast.NodeTransformer):
            def visit_Subscript(self, node):
                node = self.generic_visit(node)
                lookup = (lookups.get(node.value.id)
                          if isinstance(node.value, ast.Name) else None)
                if (lookup is not None and isinstance(node.slice, ast.Name)
                        and producers.get(node.slice.id) == lookup.index_array
                        and isinstance(node.ctx, ast.Load)):
                    name = table_for("at", lookup.name, lookup.index_array)
                    return ast.copy_location(ast.Subscript(
                        value=ast.Name(id=name, ctx=ast.Load()),
                        slice=ast.Name(id=outer_name, ctx=ast.Load()),
                        ctx=ast.Load()), node)
                return node

            def visit_Call(self, node):
                node = self.generic_visit(node)
                if not (isinstance(node.func, ast.Name)
                        and node.func.id == "_lcd_sorted_find"
                        and len(node.args) == 4):
                    return node
                index, low, high, key = node.args
                if not (isinstance(index, ast.Name)
                        and isinstance(key, ast.Name)
                        and columns.get(key.id) == index.id
                        and isinstance(low, ast.Subscript)
                        and isinstance(low.value, ast.Name)
                        and low.value.id == pointer
                        and isinstance(low.slice, ast.Name)
                        and producers.get(low.slice.id) == index.id
                        and isinstance(high, ast.Subscript)
                        and ast.unparse(high) == f"{pointer}[{low.slice.id} + 1]"):
                    return node
                # one byte per pair: the offset in the segment searched, whose
                # start is gathered by the task's own positions
                table_for("pair", pointer, index.id)
                table_for("start", pointer, index.id)
                return ast.copy_location(ast.Call(
                    func=ast.Name(id="_lcd_pair_at", ctx=ast.Load()),
                    args=[ast.Name(id=outer_name, ctx=ast.Load()),
                          ast.Name(id=inner_name, ctx=ast.Load())],
                    keywords=[]), node)

        Rewrite().visit(outer)
        ast.fix_missing_locations(outer)
        if not any(entry[0] == "pair" for entry in tables):
            # (the gathered lookup alone moves one load; not worth a table)
            pass
        for entry in tables:
            self._kinds.arrays[entry[1]] = INT
        if any(entry[0] == "pair" for entry in tables):
            self._kinds.arrays["_lcd_pair_base"] = INT
            plan["pair_row"] = True
        if tables:
            self._counted_producer_plan(body, outer, tables)
        return tuple(tables)

    def _counted_producer_plan(self, task_body, outer, tables):
        """A producer loop that opens with ``k = IDX[p]; if k >= i: break``
        runs over the leading positions of the task's own segment whose entry
        of IDX is below the task: with the segment in registers (lane l at
        position l) the wavefront finds their number with one load of IDX
        and a ballot when it takes the task, and the loop runs to that bound
        without a load and a test per producer (``plan["counted"]``).

        Every producer then is another task (``k < i``), so a position that
        comes out of a table over the producer's segment (the gathered
        lookup, the pair table) never lies in the task's own segment.  When
        every read of the array goes through the loop variables that walk
        the own segment or through such a position, the reads need not ask
        whose segment they hit and nobody reads the copy of the own segment
        in LDS (``plan["foreign"]``)."""
        plan = self._segment
        body = outer.body
        if len(body) < 2 or len(outer.iter.args) != 2:
            return
        first, leave = body[0], body[1]
        if not (isinstance(first, ast.Assign) and len(first.targets) == 1
                and isinstance(first.targets[0], ast.Name)
                and isinstance(first.value, ast.Subscript)
                and isinstance(first.value.value, ast.Name)
                and first.value.value.id not in self._all_written
                and isinstance(first.value.slice, ast.Name)
                and first.value.slice.id == outer.target.id):
            return
        producer, index_array = first.targets[0].id, first.value.value.id
        if not (isinstance(leave, ast.If) and not leave.orelse
                and len(leave.body) == 1
                and isinstance(leave.body[0], ast.Break)
                and isinstance(leave.test, ast.Compare)
                and len(leave.test.ops) == 1
                and isinstance(leave.test.ops[0], ast.GtE)
                and isinstance(leave.test.left, ast.Name)
                and leave.test.left.id == producer
                and isinstance(leave.test.comparators[0], ast.Name)
                and leave.test.comparators[0].id == self.loop_iterator):
            return
        rest = ast.Module(body=list(body[2:]), type_ignores=[])
        stores = [node.id for node in ast.walk(rest)
                  if isinstance(node, ast.Name)
                  and isinstance(node.ctx, ast.Store)]
        if producer in stores or self.loop_iterator in stores:
            return
        plan["counted"] = {
            "producer": producer, "index": index_array,
            "used": any(isinstance(node, ast.Name) and node.id == producer
                        and isinstance(node.ctx, ast.Load)
                        for node in ast.walk(rest))}
        # positions of another task's segment: the gathered lookups and the
        # pair table, both over the same index array as the loop's producers
        foreign_tables = {entry[1] for entry in tables
                          if entry[0] == "at" and entry[3] == index_array}
        pairs = any(entry[0] == "pair" and entry[3] == index_array
                    for entry in tables)
        foreign_names = {}
        for node in ast.walk(rest):
            if not isinstance(node, (ast.Assign, ast.AugAssign, ast.For)):
                continue
            targets = (node.targets if isinstance(node, ast.Assign)
                       else [node.target])
            for target in targets:
                if not isinstance(target, ast.Name):
                    continue
                value = node.value if isinstance(node, ast.Assign) else None
                good = value is not None and (
                    (isinstance(value, ast.Subscript)
                     and isinstance(value.value, ast.Name)
                     and value.value.id in foreign_tables
                     and isinstance(value.slice, ast.Name)
                     and value.slice.id == outer.target.id)
                    or (pairs and isinstance(value, ast.Call)
                        and isinstance(value.func, ast.Name)
                        and value.func.id == "_lcd_pair_at"))
                foreign_names[target.id] = (foreign_names.get(target.id, True)
                                            and good)
        others = ast.Module(body=[statement for statement in task_body
                                  if statement is not outer], type_ignores=[])
        for node in list(ast.walk(rest)) + list(ast.walk(others)):
            if (isinstance(node, ast.Subscript)
                    and isinstance(node.value, ast.Name)
                    and node.value.id == plan["array"]):
                position = node.slice
                if not isinstance(position, ast.Name):
                    return
                if position.id in plan["owned"]:
                    continue
                if not (isinstance(node.ctx, ast.Load)
                        and foreign_names.get(position.id)):
                    return
        plan["foreign"] = True

    def _segment_lines(self):
        """(prologue, epilogue) of a task that stages its own segment."""
        plan = self._segment
        array, pointer = plan["array"], plan["pointer"]
        it = self.loop_iterator
        coherent = array in self._emitter.coherent_arrays
        # with published values nobody else writes the task's own segment of
        # the array itself: its values are the input, a plain load will do
        load = (f"lcd_ld(&{array}[_lcd_seg_base + _q])"
                if coherent and not self._published
                else f"{array}[_lcd_seg_base + _q]")
        store = (f"lcd_st(&{array}[_lcd_seg_base + _q], _lcd_seg[_q]);"
                 if coherent else f"{array}[_lcd_seg_base + _q] = _lcd_seg[_q];")
        def bound(offset):
            # the copy in task order when the node loads use one
            for name, source, delta in self._queue_node_loads:
                if (source, delta) == (pointer, offset):
                    return f"{name}[_task]"
            return f"{pointer}[{it} + {offset}]" if offset else f"{pointer}[{it}]"

        if plan.get("registers"):
            # (segments longer than 64 entries are excluded by the caller; one
            # that is longer anyway stops the launch through the status word)
            plain = bool(self._published and self._published.get("plain"))
            prologue = [
                f"_lcd_seg_base = {bound(0)};",
                f"_lcd_seg_own = {bound(1)} - _lcd_seg_base;",
                # (level launches have no status word: the caller has checked
                # the segment lengths of the structure this plan is for)
                *([] if plain else
                  [f"if (_lcd_seg_own > 64) {{ {STATUS_ARGUMENT}[0] = 1; "
                   "_task_aborted = true; _lcd_seg_own = 0; }"]),
                f"_lcd_rseg = _lane < _lcd_seg_own ? {array}[_lcd_seg_base + "
                "_lane] : 0.0;",
                *([] if plan.get("foreign") else
                  ["if (_lane < _lcd_seg_own) _lcd_seg[_lane] = _lcd_rseg;"]),
                *([f"_lcd_pair_row = _lcd_pair_base[{it}];"]
                  if plan.get("pair_row") else []),
            ]
            epilogue = [
                "if (_lane < _lcd_seg_own) { lcd_pub_st(_lcd_pub, _lcd_ptile, "
                "_lcd_tpos0, _lcd_tlen, _lcd_seg_base + _lane, _lcd_rseg); "
                f"{array}[_lcd_seg_base + _lane] = _lcd_rseg; }}",
            ]
            if plain:
                epilogue = [f"if (_lane < _lcd_seg_own) "
                            f"{array}[_lcd_seg_base + _lane] = _lcd_rseg;"]
            return prologue, epilogue
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
                "lcd_pub_st(_lcd_pub, _lcd_ptile, _lcd_tpos0, _lcd_tlen, "
                "_lcd_seg_base + _q, _lcd_seg[_q]);",
                "if (_lcd_seg_limit == 0) for (int _q = _lane; _q < _lcd_seg_own; "
                "_q += LCD_TASK_LANES) lcd_pub_st(_lcd_pub, _lcd_ptile, "
                "_lcd_tpos0, _lcd_tlen, _lcd_seg_base + _q, "
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
            level = self._level_records
            if queued is not None:
                # addressed by the queue position: issued with the task id
                self._queue_load_lines.append(f"{name} = {queued}[_task];")
                if level is not None:
                    level["order"].append(
                        ("queue", f"{name} = {queued}[_task];", None))
                continue
            text = f"{name} = {emitter.expr(node)};"
            staged = self._level_value_load(name, node, text)
            if staged is not None:
                # in level order, filled by the staging kernels
                self._queue_load_lines.append(f"{name} = {staged}[_task];")
                level["order"].append(
                    ("value", f"{text} {staged}[_task] = {name};",
                     node.value.id in level["static_arrays"]))
            else:
                prefetch.append(text)
                if level is not None:
                    level["order"].append(("load", text, None))
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
        # while a queue-ordered copy is cold at every level (the same with
        # the task's producers taken flat, where the copies -- the row's
        # bounds and its place in the pair table -- save a whole dependent
        # trip: 14.4 against 13.5 ms)
        value_flags = self._value_pull is not None or (
            self._mailbox is not None and self._mailbox["gather"] is not None)
        if (not self.queue_node_loads_enabled or self.chain_tasks
                or not self.warp_mapped or not value_flags
                or (self.execution_mode != "sync_free"
                    and not self.level_gather)):
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

"""Walkers: executors in which ONE wavefront runs the tasks and nothing is
polled -- the band walker for dependence DAGs that are (nearly) a chain, the
level walker (``_level_walker_text``, at the end) for small DAGs.

Band walker.

When every level of the DAG holds about one task there is nothing to run in
parallel and a hand-off between wavefronts (a store, a poll, a load) per task
is all the persistent executor does.  The walker runs the tasks in program
order on ONE wavefront instead: lane ``t % 64`` holds task ``t``, a finished
value goes to the other lanes with two read-lanes, nothing is polled and
nothing waits.  It serves loops in the gathered mailbox form (the CSC solve:
``x[i] = f(x[i]); for j in column i: x[Ai[j]] += Ax[j] * x[i]``) and their
pull-shaped twins (the CSR solve: ``x[i] = b[i]; for j in row i: x[i] -=
Ax[j] * x[Ai[j]]; x[i] /= d``) whose edges all span fewer than 64 iterations.

What stays on the chain between two tasks is the task's own arithmetic.  The
rest of the workgroup prepares it: per block of 64 tasks the other wavefronts
write a dense table ``tab[source step][lane]`` of the coefficients (zero
where there is no edge), the node loads of every task, and the reciprocal of
a divisor that is known ahead, into LDS, one block ahead of the walker.  The
walker's step is then: finish task ``s`` (uniform operands from LDS),
broadcast its value, ``acc += tab[s][lane] * value`` in every lane.  A missing
edge adds ``0 * value``, which changes nothing while the value is finite; a
block whose values are not finite, or whose division the prepared reciprocal
does not cover, is run again with the general division and the products of
real edges only, so the result is the sequential loop's bit for bit either
way.  The reference's answer to chains is the warp task (``_band_chains``,
compiler/dag_preprocessing.py:258-298, executed by
compiler/cuda_lowering.py:1360-1410), whose members still wait on counters.
"""

import ast
import re
from copy import deepcopy

from lcd_amd.hip_emitter import FLOAT, INT, LEVEL_WALKER_TASKS

# LDS a workgroup of gfx950 can have
LDS_BYTES = 160 * 1024


class BandWalkerMixin:
    """Methods of ``HIPLowerer`` (lcd_amd/hip_lowering.py)."""

    def _band_walker_plan(self, target_loop):
        """The walker applies to the persistent executor's gathered mailbox
        when the tasks are the iterations 0 .. count - 1, the reduced array
        starts as zeros, and a product is ``operand * value`` with one
        read-only operand (a missing edge must contribute exactly nothing)."""
        box = self._mailbox
        if self.threads_per_block < 128 or self.threads_per_block % 64:
            return None      # the walker's wavefront and at least one that stages
        if (self.execution_mode != "sync_free" or box is None
                or box["gather"] is None or self.block_task
                or self.chain_tasks or len(target_loop.iter.args) != 1
                or box["array"] not in self._own_zero_arrays):
            return None
        gather = box["gather"]
        value = gather["value"]
        if len(gather["operands"]) != 1 or gather["operands"][0][2] != FLOAT:
            return None
        operand = gather["operands"][0][0]
        if not (isinstance(value, ast.BinOp) and isinstance(value.op, ast.Mult)
                and isinstance(value.left, ast.Name)
                and isinstance(value.right, ast.Name)
                and {value.left.id, value.right.id} == {operand, "_g_value"}):
            return None
        return {"operand": operand, "division": False,
                "quotient_is_value": False, "kind": "band"}

    def _band_walker_division(self, body):
        """``a / d`` with ``d`` one of the task's node loads (known a block
        ahead) becomes the tail of the division sequence over a reciprocal
        the other wavefronts prepared; the first such division only."""
        plan, lowerer = self._walker, self
        node_loads = {name for name, kind in self._kinds.locals.items()
                      if name.startswith("_nl_") and kind == FLOAT}

        class Rewrite(ast.NodeTransformer):
            def visit_BinOp(self, node):
                node = self.generic_visit(node)
                if (not plan["division"] and isinstance(node.op, ast.Div)
                        and isinstance(node.right, ast.Name)
                        and node.right.id in node_loads):
                    plan["division"] = node.right.id
                    return ast.copy_location(ast.Call(
                        func=ast.Name(id="_lcd_wdiv", ctx=ast.Load()),
                        args=[node.left, node.right], keywords=[]), node)
                return node

            def visit_AugAssign(self, node):
                node = self.generic_visit(node)
                if (not plan["division"] and isinstance(node.op, ast.Div)
                        and isinstance(node.target, ast.Name)
                        and isinstance(node.value, ast.Name)
                        and node.value.id in node_loads):
                    plan["division"] = node.value.id
                    return ast.copy_location(ast.Assign(
                        targets=[ast.Name(id=node.target.id, ctx=ast.Store())],
                        value=ast.Call(
                            func=ast.Name(id="_lcd_wdiv", ctx=ast.Load()),
                            args=[ast.Name(id=node.target.id, ctx=ast.Load()),
                                  node.value], keywords=[])), node)
                return node

        rewritten = []
        for statement in body:
            before = plan["division"]
            statement = Rewrite().visit(statement)
            if (not before and plan["division"]
                    and isinstance(statement, ast.Assign)
                    and isinstance(statement.value, ast.Call)
                    and isinstance(statement.value.func, ast.Name)
                    and statement.value.func.id == "_lcd_wdiv"
                    and len(statement.targets) == 1
                    and isinstance(statement.targets[0], ast.Name)
                    and statement.targets[0].id.startswith("_lcd_own_")):
                # the quotient is the task's value: one capture serves both
                plan["quotient_is_value"] = True
            rewritten.append(statement)
        ast.fix_missing_locations(ast.Module(body=rewritten, type_ignores=[]))
        lowerer._kinds.locals["_lcd_wr"] = FLOAT
        return rewritten

    def _prepared_division(self, body):
        """The polling executors' share of the same idea: the first ``a / d``
        whose divisor is one of the task's node loads becomes ``lcd_pdiv(a,
        d, _lcd_rcp)``, the plain division unless a pipelined fetch prepares
        the reciprocal a round ahead (LCD_PREPARED_DIVISION)."""
        lowerer = self
        node_loads = {name for name, kind in self._kinds.locals.items()
                      if name.startswith("_nl_") and kind == FLOAT}

        class Rewrite(ast.NodeTransformer):
            def visit_BinOp(self, node):
                node = self.generic_visit(node)
                if (lowerer._prepared_divisor is None
                        and isinstance(node.op, ast.Div)
                        and isinstance(node.right, ast.Name)
                        and node.right.id in node_loads):
                    lowerer._prepared_divisor = node.right.id
                    return ast.copy_location(ast.Call(
                        func=ast.Name(id="_lcd_pdiv", ctx=ast.Load()),
                        args=[node.left, node.right], keywords=[]), node)
                return node

            def visit_AugAssign(self, node):
                node = self.generic_visit(node)
                if (lowerer._prepared_divisor is None
                        and isinstance(node.op, ast.Div)
                        and isinstance(node.target, ast.Name)
                        and isinstance(node.value, ast.Name)
                        and node.value.id in node_loads):
                    lowerer._prepared_divisor = node.value.id
                    return ast.copy_location(ast.Assign(
                        targets=[ast.Name(id=node.target.id, ctx=ast.Store())],
                        value=ast.Call(
                            func=ast.Name(id="_lcd_pdiv", ctx=ast.Load()),
                            args=[ast.Name(id=node.target.id, ctx=ast.Load()),
                                  node.value], keywords=[])), node)
                return node

        rewritten = [Rewrite().visit(statement) for statement in body]
        ast.fix_missing_locations(ast.Module(body=rewritten, type_ignores=[]))
        if self._prepared_divisor is not None:
            self._kinds.locals["_lcd_rcp"] = FLOAT
            self._extra_locals.append("_lcd_rcp")
        return rewritten

    def _band_walker_store(self, lines):
        """The task's final store: the value stays in the lane (it leaves for
        memory with the block's 64 values), captured under the step's mask."""
        register = self._mailbox["register"]
        array = self._mailbox["array"]
        store = re.compile(
            r"^if \(_lane == 0\) (?:" + re.escape(array) + r"\[[^\]]*\] = "
            + re.escape(register) + r"|lcd_st\(&" + re.escape(array)
            + r"\[[^\]]*\], " + re.escape(register) + r"\));$")
        out, found = [], 0
        for line in lines:
            if store.match(line.strip()):
                found += 1
                out.append(f"_lcd_wout = {register};"
                           if self._walker.get("kind") in ("level", "sweep") else
                           f"_lcd_wout = lcd_bfi(_lcd_wmask, {register}, "
                           "_lcd_wout);")
            else:
                out.append(line)
        if found != 1:
            return None
        return out

    def _band_walker_pull_box(self, body):
        """The pull-shaped form of the same loop (the CSR solve: ``x[i] = b[i];
        for j in row i: x[i] -= Ax[j] * x[Ai[j]]; x[i] /= d``) described the
        way the gathered mailbox describes the push-shaped one, so that one
        walker serves both: the incoming listing is the row itself."""
        plan, dependence = self._value_pull, self.direct_dependence
        mapped = self._find_mapped_loop(body)
        if (plan is None or mapped is None or mapped not in body
                or len(mapped.body) != 1 or self.block_task):
            return None
        site, array = mapped.body[0], plan["array"]
        own_text = f"{array}[{self.loop_iterator}]"
        endpoint = dependence.endpoint
        if not (isinstance(site, ast.AugAssign)
                and isinstance(site.op, (ast.Add, ast.Sub))
                and ast.unparse(site.target) == own_text
                and isinstance(endpoint, ast.Subscript)
                and isinstance(endpoint.value, ast.Name)):
            return None
        kinds = self._kinds
        readonly = {name for name in kinds.arrays
                    if name not in self._all_written}
        position = mapped.target.id
        endpoint_text = ast.unparse(endpoint)

        class Substitute(ast.NodeTransformer):
            def visit_Subscript(self, node):
                if (isinstance(node.value, ast.Name) and node.value.id == array
                        and ast.unparse(node.slice) == endpoint_text):
                    return ast.Name(id="_g_value", ctx=ast.Load())
                return self.generic_visit(node)

            def visit_Name(self, node):
                if node.id == position:
                    return ast.Name(id="_g_pos", ctx=node.ctx)
                return node

        value = ast.fix_missing_locations(
            Substitute().visit(deepcopy(site.value)))
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
        for node in ast.walk(value):
            if isinstance(node, (ast.Subscript, ast.Call)):
                return None
        for name, _, kind in operands:
            kinds.locals[name] = kind
        kinds.locals["_g_value"] = FLOAT
        kinds.locals["_g_pos"] = INT
        kinds.locals["_g_src"] = INT
        return {"array": array, "position": deepcopy(endpoint.slice),
                "index_array": endpoint.value.id, "own_text": own_text,
                "sites": [site], "mapped": mapped, "pulled": True,
                "gather": {"value": value, "operands": operands, "staged": {},
                           "needs_position": True,
                           "negate": isinstance(site.op, ast.Sub)}}

    def _band_walker_text(self, task_lines):
        """Kernel body of the walker (everything after the declarations)."""
        plan = self._walker
        it = self.loop_iterator
        box = self._mailbox
        gather = box["gather"]
        emitter = self._emitter
        register = box["register"]
        array = box["array"]
        operand, operand_node, _ = gather["operands"][0]
        sign = "-" if gather["negate"] else "+"
        product = emitter.expr(gather["value"])
        # the task's text around the place of its distributed loop: what
        # comes before it gives the element its first value, what comes after
        # finishes it
        # (a push-shaped task receives its products ahead of all its own
        # statements: it has no head)
        split = plan.get("split", 0) if box.get("pulled") else 0
        head_lines, tail_lines = task_lines[:split], task_lines[split:]
        # what the other wavefronts evaluate per task: the node loads (and
        # the head); an element that starts as zero does so in the lane itself
        assign = re.compile(r"^(\w+) = (.*);$")
        stage_lines, staged, zero_start = [], [], False
        for line in self._prefetch_lines:
            match = assign.match(line.strip())
            if match is None:
                return None
            if match.group(1) == register:
                if match.group(2) != "0.0":
                    return None
                zero_start = True
                continue
            stage_lines.append(line.strip())
            staged.append(match.group(1))
        if not head_lines and not zero_start:
            return None
        for line in head_lines:
            # (whatever else the head computes for the tail is staged with
            # the node loads)
            match = assign.match(line.strip())
            if match is None:
                return None
            if match.group(1) != register:
                staged.append(match.group(1))
        tail_text = "\n".join(tail_lines)
        used = [name for name in dict.fromkeys(staged)
                if re.search(r"\b" + re.escape(name) + r"\b", tail_text)]
        slots = [(name, self._kinds.locals.get(name, FLOAT)) for name in used]
        division = plan["division"]
        if division:
            slots.append(("_lcd_wr", FLOAT))
        if head_lines:
            # (the last slot: the element's first value, taken per lane)
            slots.append((register, FLOAT))
        uniform = len(slots) - (1 if head_lines else 0)
        width = max(2, len(slots) + (len(slots) & 1))
        # (the table, the node loads, pointers, masks and flags of the ring)
        if (3 * 64 * 64 * 8 + 4 * 64 * width * 8 + 3 * 132 * 4 + 3 * 64 * 8
                + 4 * 64 * 4 > LDS_BYTES):
            return None
        own_is_quotient = bool(division) and plan["quotient_is_value"]
        general_tail = [line.replace("_lcd_wdiv(", "_lcd_wdiv_general(")
                        for line in tail_lines]
        start = (f"_w_uni[(_w_m + 1) & 3][_w_lane][{uniform}]" if head_lines
                 else "0.0")

        minus_zero = (
            f" || __double_as_longlong({register}) == (long long)0x8000000000000000ull"
            if head_lines else "")

        def put(name, kind, where):
            return (f"{where} = (double){name};" if kind == INT
                    else f"{where} = {name};")

        def take(name, kind, what):
            return (f"{name} = (lcd_index_t){what};" if kind == INT
                    else f"{name} = {what};")

        def body(lines, pad):
            return [pad + line for line in lines]

        p4, p5 = " " * 16, " " * 20
        lines = [
            "    // ---- band walker: one wavefront runs the tasks in order, the",
            "    // others stage what it needs a block of 64 tasks or two ahead",
            "    if (blockIdx.x != 0) return;",
            "    const int _w_lane = threadIdx.x & 63;",
            "    const int _w_wave = threadIdx.x >> 6;",
            "    const int _w_n = (int)task_count;",
            "    const int _w_blocks = (_w_n + 63) / 64;",
            "    const int _w_stagers = LCD_TPB - 64;",
            "    __shared__ double _w_tab[3][64][64];",
            f"    __shared__ double _w_uni[4][64][{width}];",
            "    __shared__ int _w_ptr[3][132];",
            "    __shared__ unsigned long long _w_msk[3][64];",
            "    __shared__ int _w_odd[4][64];",
            "    lcd_index_t _g_pos = 0, _g_src = 0; double _g_value = 0.0;",
            f"    double {operand} = 0.0;",
            "    double _lcd_wout = 0.0, _lcd_wq = 0.0; int _lcd_wmask = 0;",
            "    (void)_g_pos; (void)_g_src; (void)_lcd_wq;",
            "    auto _lcd_wdiv = [&](double a, double d, double r) {",
            "        const double q = lcd_div_prepared(a, d, r);",
            *([] if own_is_quotient or not division else
              ["        _lcd_wq = lcd_bfi(_lcd_wmask, q, _lcd_wq);"]),
            "        return q;",
            "    };",
            "    auto _lcd_wdiv_general = [&](double a, double d, double r) {",
            "        (void)r; return a / d;",
            "    };",
            "    (void)_lcd_wdiv; (void)_lcd_wdiv_general;",
            # ---- staging
            "    auto _w_clear = [&](int m, int first, int step) {",
            "        double* cells = &_w_tab[m % 3][0][0];",
            "        for (int c = first; c < 64 * 64; c += step) cells[c] = 0.0;",
            "        for (int c = first; c < 64; c += step) _w_msk[m % 3][c] = 0ull;",
            "    };",
            "    auto _w_stage_ptr = [&](int m, int first, int step) {",
            "        // bounds of the incoming listing of the tasks 64 m + 1 .. 64 m + 129",
            "        if (m >= _w_blocks) return;",
            "        for (int l = first; l < 130; l += step) {",
            "            const int t = m * 64 + 1 + l < _w_n ? m * 64 + 1 + l : _w_n;",
            "            _w_ptr[m % 3][l] = _lcd_in_ptr[t];",
            "        }",
            "    };",
            "    auto _w_stage = [&](int m, int first, int step) {",
            "        // the coefficients of the edges out of the tasks s0 .. s0 + 63, which",
            "        // end in s0 + 1 .. s0 + 126, by (source, lane of the destination)",
            "        if (m >= _w_blocks) return;",
            "        const int buf = m % 3, s0 = m * 64;",
            "        const int* ptr = _w_ptr[buf];",
            "        const int e0 = ptr[0], e1 = ptr[126];",
            "        for (int e = e0 + first; e < e1; e += step) {",
            "            _g_src = (lcd_index_t)_lcd_in_src[e];",
            "            if ((unsigned)(_g_src - s0) < 64u) {",
            "                _g_pos = (lcd_index_t)_lcd_in_pos[e];",
            f"                {operand} = {emitter.expr(operand_node)};",
            "                int lo = 0, hi = 126;     // the task: last l with ptr[l] <= e",
            "                while (hi - lo > 1) { const int mid = (lo + hi) >> 1; "
            "if (ptr[mid] <= e) lo = mid; else hi = mid; }",
            "                const int t = s0 + 1 + lo;",
            "                const unsigned long long bit = 1ull << (t & 63);",
            "                // an edge the table has no cell for: longer than the window, or a",
            "                // second edge between the same two tasks",
            "                if (t - _g_src >= 64 || (atomicOr(&_w_msk[buf][_g_src - s0], bit) & bit))",
            "                    _lcd_status[0] = 2;",
            f"                _w_tab[buf][_g_src - s0][t & 63] = {operand};",
            "            }",
            "        }",
            "    };",
            "    auto _w_stage_tasks = [&](int m, int first, int step) {",
            "        // per task: its node loads" + (
                ", the prepared reciprocal of its divisor" if division else "")
            + (", its element's first value" if head_lines else ""),
            "        if (m >= _w_blocks) return;",
            "        for (int l = first; l < 64; l += step) {",
            f"            {it} = (lcd_index_t)(m * 64 + l);",
            f"            if ({it} < _w_n) {{",
            *body(stage_lines, p4),
            *body(head_lines, p4),
            # (a block with a divisor the prepared reciprocal does not serve,
            # or -- pull-shaped loops -- with an element that starts as -0.0,
            # which the product of an empty cell would turn into +0.0, runs
            # again with the general division and the products of real edges)
            *([f"{p4}_lcd_wr = lcd_div_prepare({division});",
               f"{p4}_w_odd[m & 3][l] = !lcd_div_plain_divisor({division}){minus_zero};"]
              if division else [f"{p4}_w_odd[m & 3][l] = 0{minus_zero};"]),
            *[p4 + put(name, kind, f"_w_uni[m & 3][l][{k}]")
              for k, (name, kind) in enumerate(slots)],
            "            }",
            "        }",
            "    };",
            "    _w_clear(0, threadIdx.x, LCD_TPB); _w_clear(1, threadIdx.x, LCD_TPB); "
            "_w_clear(2, threadIdx.x, LCD_TPB);",
            "    _w_stage_ptr(0, threadIdx.x, LCD_TPB); _w_stage_ptr(1, threadIdx.x, LCD_TPB);",
            "    _w_stage_tasks(0, threadIdx.x, LCD_TPB); _w_stage_tasks(1, threadIdx.x, LCD_TPB);",
            "    __syncthreads();",
            "    _w_stage(0, threadIdx.x, LCD_TPB);",
            "    __syncthreads();",
            (f"    {register} = _w_uni[0][_w_lane][{uniform}];" if head_lines
             else f"    {register} = 0.0;"),
            "    for (int _w_m = 0; _w_m < _w_blocks; ++_w_m) {",
            "        if (_w_wave == 0) {",
            "            const int base = _w_m * 64;",
            "            const int steps = _w_n - base < 64 ? _w_n - base : 64;",
            "            const int cb = _w_m % 3, ub = _w_m & 3;",
            f"            const double _w_acc0 = {register};",
            # the value the lane's next task (64 later) starts from
            f"            const double _w_start = {start};",
            "            _lcd_wmask = _w_lane == 0 ? -1 : 0;",
            "            if (steps == 64) {",
            "                double _w_w = _w_tab[cb][0][_w_lane];",
            *[f"{p4}double _w_u{k} = _w_uni[ub][0][{k}];"
              for k in range(uniform)],
            "#pragma unroll 4",
            "                for (int l = 0; l < 64; ++l) {",
            "                    const int ln = (l + 1) & 63;",
            f"                    {it} = (lcd_index_t)(base + l);",
            *[p5 + take(name, kind, f"_w_u{k}")
              for k, (name, kind) in enumerate(slots[:uniform])],
            f"                    const double _w_acc = {register};",
            *body(tail_lines, p5),
            f"                    const double _w_xs = lcd_rseg_uni({register}, (lcd_index_t)l);",
            "                    const double _w_wn = _w_tab[cb][ln][_w_lane];",
            *[f"{p5}const double _w_n{k} = _w_uni[ub][ln][{k}];"
              for k in range(uniform)],
            # the lane of the finished task starts its next one; its cell of
            # this row is empty
            f"                    {register} = lcd_bfi(_lcd_wmask, _w_start, _w_acc);",
            "                    _lcd_wmask = lcd_next_lane(_lcd_wmask);",
            f"                    _g_value = _w_xs; {operand} = _w_w;",
            f"                    {register} = {register} {sign} {product};",
            "                    _w_w = _w_wn;",
            *[f"{p5}_w_u{k} = _w_n{k};" for k in range(uniform)],
            "                }",
            "            }",
            # the check and the second, general pass
            "            bool _w_again = steps < 64;",
            (f"            _w_again = _w_again || __ballot(_w_odd[ub][_w_lane] != 0 "
             f"|| !lcd_div_plain_quotient("
             f"{'_lcd_wout' if own_is_quotient else '_lcd_wq'}) "
             "|| !lcd_finite(_lcd_wout)) != 0ull;" if division else
             "            _w_again = _w_again || __ballot(_w_odd[ub][_w_lane] != 0 "
             "|| !lcd_finite(_lcd_wout)) != 0ull;"),
            "            if (_w_again) {",
            "                // the general division, and the products of real edges only",
            f"                {register} = _w_acc0;",
            "                _lcd_wmask = _w_lane == 0 ? -1 : 0;",
            "                for (int l = 0; l < steps; ++l) {",
            f"                    {it} = (lcd_index_t)(base + l);",
            *[p5 + take(name, kind, f"_w_uni[ub][l][{k}]")
              for k, (name, kind) in enumerate(slots[:uniform])],
            f"                    const double _w_acc = {register};",
            *body(general_tail, p5),
            f"                    const double _w_xs = lcd_rseg_uni({register}, (lcd_index_t)l);",
            f"                    {register} = lcd_bfi(_lcd_wmask, _w_start, _w_acc);",
            "                    _lcd_wmask = lcd_next_lane(_lcd_wmask);",
            "                    if ((_w_msk[cb][l] >> _w_lane) & 1ull) {",
            f"                        _g_value = _w_xs; {operand} = _w_tab[cb][l][_w_lane];",
            f"                        {register} = {register} {sign} {product};",
            "                    }",
            "                }",
            "            }",
            f"            if (_w_lane < steps) {array}[base + _w_lane] = _lcd_wout;",
            "        } else {",
            "            const int first = threadIdx.x - 64;",
            "            _w_stage(_w_m + 1, first, _w_stagers);",
            "            _w_clear(_w_m + 2, first, _w_stagers);",
            "            _w_stage_ptr(_w_m + 2, first, _w_stagers);",
            "            _w_stage_tasks(_w_m + 2, first, _w_stagers);",
            "        }",
            "        __syncthreads();",
            "    }",
        ]
        return lines

    # ---- the level walker: small DAGs with narrow levels
    def _level_walker_text(self, task_lines):
        """Kernel body for a DAG of at most LCD_LW_TASKS tasks whose levels
        hold at most 64 of them and whose tasks have at most LCD_LW_ENTRIES
        incoming entries: ONE wavefront takes a level per step, one task per
        lane.  The values live in LDS; a level's reads follow the stores of
        the levels before it in program order, so nothing is polled.  The
        structure comes level-major from the inspector (``_lcd_lw_task``: the
        task of (level, lane) or -1; ``_lcd_lw_src`` / ``_lcd_lw_pos``: the
        source and the operand position of its k-th incoming entry, in the
        listing's order, or the dummy slot / -1); the other wavefronts gather
        operands and node loads into an LDS ring, blocks of eight levels, two
        blocks ahead.  No arithmetic differs from the sequential loop's."""
        plan = self._walker
        it = self.loop_iterator
        box = self._mailbox
        gather = box["gather"]
        emitter = self._emitter
        register = box["register"]
        array = box["array"]
        operand, operand_node, _ = gather["operands"][0]
        sign = "-" if gather["negate"] else "+"
        product = emitter.expr(gather["value"])
        entries = int(plan["entries"])
        split = plan.get("split", 0) if box.get("pulled") else 0
        head_lines, tail_lines = task_lines[:split], task_lines[split:]
        assign = re.compile(r"^(\w+) = (.*);$")
        stage_lines, staged, zero_start = [], [], False
        for line in self._prefetch_lines:
            match = assign.match(line.strip())
            if match is None:
                return None
            if match.group(1) == register:
                if match.group(2) != "0.0":
                    return None
                zero_start = True
                continue
            stage_lines.append(line.strip())
            staged.append(match.group(1))
        if not head_lines and not zero_start:
            return None
        for line in head_lines:
            match = assign.match(line.strip())
            if match is None:
                return None
            if match.group(1) != register:
                staged.append(match.group(1))
        tail_text = "\n".join(tail_lines)
        slots = [(name, self._kinds.locals.get(name, FLOAT))
                 for name in dict.fromkeys(staged)
                 if re.search(r"\b" + re.escape(name) + r"\b", tail_text)]
        division = plan["division"]
        if division:
            # (the prepared reciprocal of the task's divisor, per lane; not a
            # number where the divisor is outside the range it serves)
            slots.append(("_lcd_wr", FLOAT))
        if head_lines:
            slots.append((register, FLOAT))
        width = max(1, len(slots))
        # (the values, then three blocks of eight levels: operands, sources,
        # node loads and tasks)
        if ((LEVEL_WALKER_TASKS + 2) * 8 + 3 * 8 * 64 * (
                entries * (8 + 2) + width * 8 + 4) > LDS_BYTES):
            return None
        general_tail = [line.replace("_lcd_wdiv(", "_lcd_wdiv_general(")
                        for line in tail_lines]

        def put(name, kind, where):
            return (f"{where} = (double){name};" if kind == INT
                    else f"{where} = {name};")

        def take(name, kind, what):
            return (f"{name} = (lcd_index_t){what};" if kind == INT
                    else f"{name} = {what};")

        p3, p4 = " " * 12, " " * 16

        def steps(tail):
            return [
            "            int _w_t = _w_task[rb][0][_w_lane];",
            "            short _w_s[LW_K]; double _w_c[LW_K];",
            f"            double _w_u[{width}];",
            "#pragma unroll",
            "            for (int k = 0; k < LW_K; ++k) { _w_s[k] = _w_src[rb][0][k][_w_lane]; "
            "_w_c[k] = _w_coef[rb][0][k][_w_lane]; }",
            "#pragma unroll",
            f"            for (int k = 0; k < {width}; ++k) _w_u[k] = _w_uni[rb][0][k][_w_lane];",
            "#pragma unroll 2",
            "            for (int l = 0; l < LW_B; ++l) {",
            "                const int ln = l + 1 < LW_B ? l + 1 : l;",
            "                const int task = _w_t;",
            "                double _w_v[LW_K];",
            "#pragma unroll",
            "                for (int k = 0; k < LW_K; ++k) _w_v[k] = _w_x[_w_s[k]];",
            f"                {it} = (lcd_index_t)(task < 0 ? 0 : task);",
            f"                {register} = " + (f"_w_u[{len(slots) - 1}]" if head_lines else "0.0") + ";",
            *[p4 + take(name, kind, f"_w_u[{k}]")
              for k, (name, kind) in enumerate(slots)
              if not (head_lines and k == len(slots) - 1)],
            "                double _w_cc[LW_K];",
            "#pragma unroll",
            "                for (int k = 0; k < LW_K; ++k) _w_cc[k] = _w_c[k];",
            "                _w_t = _w_task[rb][ln][_w_lane];",
            "#pragma unroll",
            "                for (int k = 0; k < LW_K; ++k) { _w_s[k] = _w_src[rb][ln][k][_w_lane]; "
            "_w_c[k] = _w_coef[rb][ln][k][_w_lane]; }",
            "#pragma unroll",
            f"                for (int k = 0; k < {width}; ++k) _w_u[k] = _w_uni[rb][ln][k][_w_lane];",
            "#pragma unroll",
            "                for (int k = 0; k < LW_K; ++k) {",
            f"                    _g_value = _w_v[k]; {operand} = _w_cc[k];",
            f"                    {register} = {register} {sign} {product};",
            "                }",
            *[p4 + line for line in tail],
            # (a lane without a task writes the slot nobody reads: no branch
            # between the division and the store)
            "                _w_x[task < 0 ? LCD_LW_TASKS + 1 : task] = _lcd_wout;",
            "            }",
            ]

        first_value = (f"_w_uni[rb][l][{len(slots) - 1}][_w_lane]" if head_lines
                       else "0.0")
        lines = [
            "    // ---- level walker: one wavefront takes a level per step",
            "    if (blockIdx.x != 0) return;",
            "    const int _w_lane = threadIdx.x & 63;",
            "    const int _w_wave = threadIdx.x >> 6;",
            "    const int _w_n = (int)task_count;",
            f"    constexpr int LW_K = {entries}, LW_B = 8;",
            "    const int _w_levels = (int)_lcd_lw_levels;",
            "    const int _w_blocks = (_w_levels + LW_B - 1) / LW_B;",
            "    const int _w_helpers = LCD_TPB - 64;",
            "    __shared__ double _w_x[LCD_LW_TASKS + 2];",
            "    __shared__ double _w_coef[3][LW_B][LW_K][64];",
            "    __shared__ short _w_src[3][LW_B][LW_K][64];",
            f"    __shared__ double _w_uni[3][LW_B][{width}][64];",
            "    __shared__ int _w_task[3][LW_B][64];",
            "    lcd_index_t _g_pos = 0, _g_src = 0; double _g_value = 0.0;",
            f"    double {operand} = 0.0; double _lcd_wout = 0.0;",
            "    unsigned _lcd_wbad = 0; (void)_lcd_wbad;",
            "    (void)_g_pos; (void)_g_src;",
            # the division over the prepared reciprocal; how far its quotient is
            # from the range in which that is the division is kept per lane and
            # looked at once per block
            "    auto _lcd_wdiv = [&](double a, double d, double r) {",
            "        const double q = lcd_div_prepared(a, d, r);",
            "        const unsigned off = ((((unsigned)(__double_as_longlong(q) >> 32)) >> 20) "
            "& 0x7ffu) - 164u;",
            "        _lcd_wbad = off > _lcd_wbad ? off : _lcd_wbad;",
            "        return q;",
            "    };",
            "    auto _lcd_wdiv_general = [&](double a, double d, double r) {",
            "        (void)r; return a / d;",
            "    };",
            "    (void)_lcd_wdiv; (void)_lcd_wdiv_general;",
            "    if (_w_n > LCD_LW_TASKS) { if (threadIdx.x == 0) _lcd_status[0] = 2; return; }",
            "    auto _w_stage = [&](int m, int first, int step) {",
            "        // block m of the levels: tasks, node loads, sources and operands",
            "        if (m >= _w_blocks) return;",
            "        const int rb = m % 3;",
            "        for (int c = first; c < LW_B * 64; c += step) {",
            "            const int l = c >> 6, lane = c & 63, level = m * LW_B + l;",
            "            const int task = level < _w_levels ? "
            "(int)_lcd_lw_task[level * 64 + lane] : -1;",
            "            _w_task[rb][l][lane] = task;",
            # (a lane without a task computes on ones: nothing out of range)
            f"            for (int k = 0; k < {width}; ++k) _w_uni[rb][l][k][lane] = 1.0;",
            "            if (task >= 0) {",
            f"                {it} = (lcd_index_t)task;",
            *[p4 + line for line in stage_lines],
            *[p4 + line for line in head_lines],
            *([f"{p4}_lcd_wr = lcd_div_plain_divisor({division}) ? "
               f"lcd_div_prepare({division}) : lcd_empty();"]
              if division else []),
            *[p4 + put(name, kind, f"_w_uni[rb][l][{k}][lane]")
              for k, (name, kind) in enumerate(slots)],
            "            }",
            "        }",
            "        for (int c = first; c < LW_B * LW_K * 64; c += step) {",
            "            const int lane = c & 63, k = (c >> 6) % LW_K, l = c / (64 * LW_K);",
            "            const int level = m * LW_B + l;",
            # (x + -0.0 and x - +0.0 leave every x as it is, signed zeros included)
            "            int src = LCD_LW_TASKS; double coef = "
            + ("-0.0" if sign == "+" else "0.0") + ";",
            "            if (level < _w_levels) {",
            "                const long long at = ((long long)level * LW_K + k) * 64 + lane;",
            "                _g_pos = (lcd_index_t)_lcd_lw_pos[at];",
            "                if (_g_pos >= 0) {",
            "                    _g_src = (lcd_index_t)_lcd_lw_src[at]; src = (int)_g_src;",
            f"                    coef = {emitter.expr(operand_node)};",
            "                }",
            "            }",
            "            _w_src[rb][l][k][lane] = (short)src;",
            "            _w_coef[rb][l][k][lane] = coef;",
            "        }",
            "    };",
            "    // (an entry that is not there reads the slot past the last task, which",
            "    // holds zero, with a zero operand)",
            "    for (int c = threadIdx.x; c < LCD_LW_TASKS + 1; c += LCD_TPB) _w_x[c] = 0.0;",
            "    _w_stage(0, threadIdx.x, LCD_TPB); _w_stage(1, threadIdx.x, LCD_TPB);",
            "    __syncthreads();",
            "    for (int _w_m = 0; _w_m < _w_blocks; ++_w_m) {",
            "        if (_w_wave == 0) {",
            "            const int rb = _w_m % 3;",
            "            _lcd_wbad = 0;",
            # what a level reads from the ring is in registers a level ahead:
            # the step then waits for one trip to LDS (the sources' values)
            *steps(tail_lines),
            *([
                "            if (__ballot(_lcd_wbad > 1518u) != 0ull) {",
                "                // a quotient (or a divisor) the prepared reciprocal does not",
                "                // serve: the block again with the general division",
                *["    " + line for line in steps(general_tail)],
                "            }",
            ] if division else []),
            "        } else {",
            "            _w_stage(_w_m + 2, threadIdx.x - 64, _w_helpers);",
            "        }",
            "        __syncthreads();",
            "    }",
            # the values leave LDS together, every thread of the workgroup a few
            f"    for (int c = threadIdx.x; c < _w_n; c += LCD_TPB) {array}[c] = _w_x[c];",
        ]
        return lines

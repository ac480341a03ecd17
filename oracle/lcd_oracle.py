"""ctypes front end of ``liblcd_oracle.so`` plus literal Python restatements.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Two layers:

* ``literal_*``: line-for-line pure-Python restatements of what the
  reference executes (set-based inspector, Kahn wavefronts, the user loops).
  They are slow and only used on small inputs to pin the C oracle.
* everything else: thin wrappers over the C oracle, usable at full size.
"""

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblcd_oracle.so")
_lib = None

GUARD_NONE, GUARD_GREATER, GUARD_NOT_EQUAL = 0, 1, 2


class _Rule(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("idx", ctypes.c_void_p),
        ("owner_is_source", ctypes.c_int32),
        ("lower_offset", ctypes.c_int32),
        ("upper_offset", ctypes.c_int32),
        ("guard", ctypes.c_int32),
        ("break_at_owner", ctypes.c_int32),
        ("relation", ctypes.c_int32),
    ]


class _Dag(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int64),
        ("edges", ctypes.c_int64),
        ("levels", ctypes.c_int64),
        ("scheduled", ctypes.c_int64),
        ("dag_ptr", ctypes.POINTER(ctypes.c_int32)),
        ("dag_index", ctypes.POINTER(ctypes.c_int32)),
        ("dep_count", ctypes.POINTER(ctypes.c_int32)),
        ("edge_count", ctypes.POINTER(ctypes.c_int32)),
        ("level_of", ctypes.POINTER(ctypes.c_int32)),
        ("wavefronts", ctypes.POINTER(ctypes.c_int32)),
        ("wavefront_ptr", ctypes.POINTER(ctypes.c_int32)),
        ("status", ctypes.c_int32),
    ]


def build(force=False):
    """Compile the C oracle in place (gcc, seconds)."""
    if force or not os.path.exists(_LIB_PATH) or (
            os.path.getmtime(_LIB_PATH)
            < os.path.getmtime(os.path.join(_HERE, "lcd_oracle.c"))):
        subprocess.run(["make", "-C", _HERE, "-s", "-B"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.oracle_dag_build.restype = ctypes.POINTER(_Dag)
        _lib.oracle_dag_build.argtypes = [
            ctypes.POINTER(_Rule), ctypes.c_int32, ctypes.c_int64]
        _lib.oracle_dag_from_successors.restype = ctypes.POINTER(_Dag)
        _lib.oracle_dag_from_successors.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
        _lib.oracle_dag_free.argtypes = [ctypes.POINTER(_Dag)]
        _lib.oracle_dag_free.restype = None
        _lib.oracle_band_chains.restype = ctypes.c_int64
        _lib.oracle_band_chains.argtypes = [
            ctypes.POINTER(_Dag), ctypes.c_int64, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_void_p]
        _lib.oracle_lookup_positions.restype = ctypes.c_int32
        _lib.oracle_ilu0_csr_flops.restype = ctypes.c_int64
    return _lib


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _f64(a):
    return np.ascontiguousarray(a, dtype=np.float64)


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


# ------------------------------------------------------------------ solvers

def sptrsv_csc(Ap, Ai, Ax, b, n):
    Ap, Ai, Ax, b = _i32(Ap), _i32(Ai), _f64(Ax), _f64(b)
    x = np.empty(n, dtype=np.float64)
    lib().oracle_sptrsv_csc(_p(Ap), _p(Ai), _p(Ax), _p(b),
                            ctypes.c_int64(n), _p(x))
    return x


def sptrsv_csr(Ap, Ai, Ax, b, n):
    Ap, Ai, Ax, b = _i32(Ap), _i32(Ai), _f64(Ax), _f64(b)
    x = np.empty(n, dtype=np.float64)
    lib().oracle_sptrsv_csr(_p(Ap), _p(Ai), _p(Ax), _p(b),
                            ctypes.c_int64(n), _p(x))
    return x


def gauss_seidel_csr(Ap, Ai, Ax, D, b, x, n, max_iter):
    Ap, Ai, Ax, D, b = _i32(Ap), _i32(Ai), _f64(Ax), _f64(D), _f64(b)
    x = _f64(x).copy()
    lib().oracle_gauss_seidel_csr(_p(Ap), _p(Ai), _p(Ax), _p(D), _p(b), _p(x),
                                  ctypes.c_int64(n), ctypes.c_int64(max_iter))
    return x


def ilu0_csr(A_data, A_indices, A_indptr):
    data = _f64(A_data).copy()
    idx, ptr = _i32(A_indices), _i32(A_indptr)
    lib().oracle_ilu0_csr(_p(data), _p(idx), _p(ptr),
                          ctypes.c_int64(len(ptr) - 1))
    return data


def ilu0_csc(A_data, A_indices, A_indptr):
    data = _f64(A_data).copy()
    idx, ptr = _i32(A_indices), _i32(A_indptr)
    lib().oracle_ilu0_csc(_p(data), _p(idx), _p(ptr),
                          ctypes.c_int64(len(ptr) - 1))
    return data


def ilu0_csr_flops(A_indices, A_indptr):
    idx, ptr = _i32(A_indices), _i32(A_indptr)
    return int(lib().oracle_ilu0_csr_flops(_p(idx), _p(ptr),
                                           ctypes.c_int64(len(ptr) - 1)))


# ---------------------------------------------------------------------- DAG

class Dag:
    """NumPy copies of one oracle DAG."""

    def __init__(self, handle):
        d = handle.contents
        self.n, self.edges = int(d.n), int(d.edges)
        self.levels, self.scheduled = int(d.levels), int(d.scheduled)
        self.status = int(d.status)

        def take(pointer, count):
            if not pointer or count == 0:
                return np.zeros(0, dtype=np.int32)
            return np.ctypeslib.as_array(pointer, shape=(count,)).copy()

        n = self.n
        self.dag_ptr = take(d.dag_ptr, n + 1)
        self.edge_count = take(d.edge_count, n)
        self.dep_count = take(d.dep_count, n)
        if self.status == 0:
            self.dag_index = take(d.dag_index, self.edges)
            self.level_of = take(d.level_of, n)
            self.wavefronts = take(d.wavefronts, self.scheduled)
            self.wavefront_ptr = take(d.wavefront_ptr, self.levels + 1)
        self._handle = handle

    def band_chains(self, band_width):
        bands = -(-self.levels // band_width)
        task_nodes = np.empty(max(self.n, 1), dtype=np.int32)
        task_ptr = np.empty(self.n + 1, dtype=np.int32)
        band_ptr = np.empty(bands + 1, dtype=np.int32)
        tasks = lib().oracle_band_chains(
            self._handle, ctypes.c_int64(band_width), _p(task_nodes),
            _p(task_ptr), _p(band_ptr))
        return task_nodes[:self.n], task_ptr[:tasks + 1], band_ptr

    def successors(self):
        return [
            self.dag_index[self.dag_ptr[v]:self.dag_ptr[v + 1]].tolist()
            for v in range(self.n)
        ]

    def wavefront_list(self):
        return [
            self.wavefronts[
                self.wavefront_ptr[k]:self.wavefront_ptr[k + 1]].tolist()
            for k in range(self.levels)
        ]

    def __del__(self):
        try:
            lib().oracle_dag_free(self._handle)
        except Exception:
            pass


def make_rule(ptr, idx, owner_is_source, lower_offset=0, upper_offset=0,
              guard=GUARD_GREATER, break_at_owner=False):
    return dict(ptr=_i32(ptr), idx=_i32(idx),
                owner_is_source=bool(owner_is_source),
                lower_offset=int(lower_offset), upper_offset=int(upper_offset),
                guard=int(guard), break_at_owner=bool(break_at_owner))


#: edge rules of the supported loops, as the reference's planner derives them
#: (compiler/transform_tests/test_dag_codegen.py:58-99,
#:  test_spilu0_codegen.py:129-144, test_gauss_seidel_codegen.py:143-148).
def rule_sptrsv_csc(Ap, Ai):
    return make_rule(Ap, Ai, True, lower_offset=1, guard=GUARD_GREATER)


def rule_sptrsv_csr(Ap, Ai):
    return make_rule(Ap, Ai, False, upper_offset=-1, guard=GUARD_GREATER)


def rule_gauss_seidel_csr(Ap, Ai):
    return make_rule(Ap, Ai, False, guard=GUARD_GREATER)


def rule_ilu0_csr(A_indptr, A_indices):
    return make_rule(A_indptr, A_indices, False, guard=GUARD_NONE,
                     break_at_owner=True)


def rule_later(lower_offset=1):
    """``for j in range(seg + lower_offset, n)``: seg -> j."""
    return dict(relation=1, lower_offset=int(lower_offset))


def rule_next(lower_offset=1):
    """The chain rule: seg -> seg + lower_offset."""
    return dict(relation=2, lower_offset=int(lower_offset))


def rules_ilu0_csc(A_indptr, A_indices):
    """The two rules of CSC ILU0
    (compiler/transform_tests/test_spilu0_codegen.py:146-150)."""
    return [make_rule(A_indptr, A_indices, True, guard=GUARD_GREATER),
            rule_later(1)]


def dag_build(rules, n):
    rules = list(rules)
    array = (_Rule * len(rules))()
    keep = []
    for slot, rule in zip(array, rules):
        if rule.get("relation"):
            slot.relation = int(rule["relation"])
            slot.lower_offset = rule["lower_offset"]
            continue
        keep.append((rule["ptr"], rule["idx"]))
        slot.ptr = rule["ptr"].ctypes.data
        slot.idx = rule["idx"].ctypes.data
        slot.owner_is_source = int(rule["owner_is_source"])
        slot.lower_offset = rule["lower_offset"]
        slot.upper_offset = rule["upper_offset"]
        slot.guard = rule["guard"]
        slot.break_at_owner = int(rule["break_at_owner"])
    return Dag(lib().oracle_dag_build(array, len(rules), ctypes.c_int64(n)))


def dag_from_successors(successors):
    n = len(successors)
    ptr = np.zeros(n + 1, dtype=np.int32)
    flat = []
    for v, nbrs in enumerate(successors):
        flat.extend(int(w) for w in nbrs)
        ptr[v + 1] = len(flat)
    index = np.asarray(flat, dtype=np.int32)
    return Dag(lib().oracle_dag_from_successors(_p(ptr), _p(index),
                                                ctypes.c_int64(n)))


def lookup_positions(ptr, idx):
    ptr, idx = _i32(ptr), _i32(idx)
    n = len(ptr) - 1
    out = np.empty(max(n, 0), dtype=np.int32)
    status = lib().oracle_lookup_positions(
        _p(ptr), _p(idx), ctypes.c_int64(n), ctypes.c_int64(len(idx)), _p(out))
    return int(status), out


# ---------------------------------------- literal pure-Python restatements

def literal_extract_dag(rule, n, execution_mode="sync_free",
                        edge_multiplicity=False):
    """The generated ``extract_dag`` for one rule, or a list of rules,
    statement by statement (compiler/dag_codegen.py:1164-1196, 1484-1505)."""
    successors = [set() for _ in range(n)]
    edge_count = [0 for _ in range(n)]
    for rule in (rule if isinstance(rule, (list, tuple)) else [rule]):
        if rule.get("relation") == 2:
            for seg in range(0, n - rule["lower_offset"]):
                successors[seg].add(seg + rule["lower_offset"])
                edge_count[seg + rule["lower_offset"]] += 1
            continue
        if rule.get("relation"):
            for seg in range(0, n):
                for later in range(seg + rule["lower_offset"], n):
                    successors[seg].add(later)
                    edge_count[later] += 1
            continue
        ptr, idx = rule["ptr"].tolist(), rule["idx"].tolist()
        for seg in range(0, n):
            for p in range(ptr[seg] + rule["lower_offset"],
                           ptr[seg + 1] + rule["upper_offset"]):
                if rule["break_at_owner"] and idx[p] >= seg:
                    break
                if rule["owner_is_source"]:
                    source, destination = seg, idx[p]
                else:
                    source, destination = idx[p], seg
                if rule["guard"] == GUARD_GREATER and not destination > source:
                    continue
                if rule["guard"] == GUARD_NOT_EQUAL and source == destination:
                    continue
                successors[source].add(destination)
                edge_count[destination] += 1
    dep_count = [0 for _ in range(n)]
    for neighbours in successors:
        for destination in neighbours:
            dep_count[destination] += 1
    dag = [sorted(neighbours) for neighbours in successors]
    if execution_mode == "wavefront":
        scheduling = literal_wavefronts_from_dag(dag, dep_count)
    else:
        scheduling = dep_count
    if edge_multiplicity:
        return dag, scheduling, edge_count
    return dag, scheduling


def literal_wavefronts_from_dag(dag_successors, dep_count):
    """compiler/dag_preprocessing.py:146-163."""
    remaining = list(dep_count)
    wavefront_list = []
    wavefront = [node for node, count in enumerate(remaining) if count == 0]
    while wavefront:
        wavefront_list.append(wavefront)
        new_wavefront = set()
        for node in wavefront:
            for successor in dag_successors[node]:
                remaining[successor] -= 1
                if remaining[successor] == 0:
                    new_wavefront.add(successor)
        wavefront = sorted(new_wavefront)
    return wavefront_list


def literal_band_chains(nodes, level_ptr, dag_ptr, dag_index, band_width):
    """compiler/dag_preprocessing.py:258-298 (union-find per band)."""
    level_count = len(level_ptr) - 1
    task_nodes, task_ptr, band_ptr = [], [0], [0]
    for first_level in range(0, level_count, band_width):
        last_level = min(first_level + band_width, level_count)
        band = list(nodes[level_ptr[first_level]:level_ptr[last_level]])
        local = {node: position for position, node in enumerate(band)}
        parent = list(range(len(band)))

        def find(position):
            while parent[position] != position:
                position = parent[position]
            return position

        for position, node in enumerate(band):
            for successor in dag_index[dag_ptr[node]:dag_ptr[node + 1]]:
                successor_position = local.get(int(successor))
                if successor_position is not None:
                    root, other = find(position), find(successor_position)
                    if root != other:
                        parent[other] = root
        chains = {}
        for position, node in enumerate(band):
            chains.setdefault(find(position), []).append(int(node))
        for chain in chains.values():
            task_nodes.extend(chain)
            task_ptr.append(len(task_nodes))
        band_ptr.append(len(task_ptr) - 1)
    return task_nodes, task_ptr, band_ptr


def literal_sptrsv_csc(Ap, Ai, Ax, b, n):
    """README.md:85-92."""
    x = np.zeros(n)
    for i in range(n):
        x[i] = (b[i] - x[i]) / Ax[Ap[i]]
        for j in range(Ap[i] + 1, Ap[i + 1]):
            x[Ai[j]] += Ax[j] * x[i]
    return x


def literal_sptrsv_csr(Ap, Ai, Ax, b, n):
    """compiler/demo/sptrsv.py:26-33."""
    x = np.zeros(n)
    for i in range(n):
        x[i] = b[i]
        for j in range(Ap[i], Ap[i + 1] - 1):
            x[i] -= Ax[j] * x[Ai[j]]
        x[i] /= Ax[Ap[i + 1] - 1]
    return x


def literal_ilu0_csr(A_data, A_indices, A_indptr):
    """compiler/demo/spilu0.py:21-47."""
    n = len(A_indptr) - 1
    for i in range(n):
        row_start = A_indptr[i]
        row_end = A_indptr[i + 1]
        for k_ptr in range(row_start, row_end):
            k = A_indices[k_ptr]
            if k >= i:
                break
            diag_val = 0.0
            for diag_ptr in range(A_indptr[k], A_indptr[k + 1]):
                if A_indices[diag_ptr] == k:
                    diag_val = A_data[diag_ptr]
                    break
            if diag_val != 0.0:
                A_data[k_ptr] = A_data[k_ptr] / diag_val
                l_ik = A_data[k_ptr]
                for j_ptr in range(k_ptr + 1, row_end):
                    j = A_indices[j_ptr]
                    for kj_ptr in range(A_indptr[k], A_indptr[k + 1]):
                        if A_indices[kj_ptr] == j:
                            u_kj = A_data[kj_ptr]
                            A_data[j_ptr] = A_data[j_ptr] - l_ik * u_kj
                            break
    return A_data

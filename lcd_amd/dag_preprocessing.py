"""Executor data structures built from an inspected DAG.

Mirrors compiler/dag_preprocessing.py of the reference.  The `@parallel`
path never runs the host functions below: it gets the same arrays from the
on-device inspector (``execution_data_from_device_dag``).  The list-based
functions keep the reference's public interface for callers that hold Python
successor lists (``wrapper.build_dag`` output, hand-built DAGs); they validate
exactly what the reference validates and are vectorised with NumPy.
"""

from dataclasses import dataclass, field, replace

import numpy as np


class DAGPreprocessingError(Exception):
    """Generated DAG data cannot form executor inputs."""


@dataclass(frozen=True)
class SyncFreeExecutionData:
    """CSR successors and mutable incoming-dependency counts."""

    dep_count: object
    dag_ptr: object
    dag_index: object
    initial_dep_count: object = None
    auxiliary_values: dict = field(default_factory=dict)

    @property
    def launcher_arguments(self):
        return self.dep_count, self.dag_ptr, self.dag_index


@dataclass(frozen=True)
class WavefrontExecutionData:
    """Flattened wavefront nodes and offsets for each wavefront."""

    wavefronts: object
    wavefront_ptr: object
    auxiliary_values: dict = field(default_factory=dict)

    @property
    def launcher_arguments(self):
        return self.wavefronts, self.wavefront_ptr


@dataclass(frozen=True)
class WarpTaskExecutionData:
    """Task lists for group-mapped executors (one wavefront or a slice of one
    per task)."""

    task_nodes: object
    task_ptr: object
    band_ptr: object
    dep_count: object
    dag_ptr: object
    dag_index: object
    initial_dep_count: object = None
    auxiliary_values: dict = field(default_factory=dict)


def preprocess_dag_output(dag_successors, scheduling_data, execution_mode):
    """Convert inspector output to the selected executor format."""
    execution_mode = execution_mode.replace("-", "_")
    if execution_mode == "sync_free":
        return preprocess_sync_free(dag_successors, scheduling_data)
    if execution_mode == "wavefront":
        return preprocess_wavefront(dag_successors, scheduling_data)
    raise DAGPreprocessingError(
        f"Unknown execution mode {execution_mode!r}; expected sync_free "
        "or wavefront.")


def attach_auxiliary_values(execution_data, auxiliary_values):
    """Attach immutable inspector outputs (lookup tables) to executor data."""
    if not auxiliary_values:
        return execution_data
    if not isinstance(execution_data, (SyncFreeExecutionData,
                                       WavefrontExecutionData,
                                       WarpTaskExecutionData)):
        raise DAGPreprocessingError(
            "Auxiliary values require recognized DAG execution data.")
    collisions = set(execution_data.auxiliary_values) & set(auxiliary_values)
    if collisions:
        raise DAGPreprocessingError(
            "Duplicate auxiliary execution values: "
            + ", ".join(sorted(collisions)))
    combined = dict(execution_data.auxiliary_values)
    combined.update(auxiliary_values)
    return replace(execution_data, auxiliary_values=combined)


def compact_successors(dag_successors):
    """Successor lists -> CSR ``dag_ptr``/``dag_index`` (sorted, unique)."""
    node_count = len(dag_successors)
    dag_ptr = np.zeros(node_count + 1, dtype=np.int32)
    pieces = []
    for source, successors in enumerate(dag_successors):
        try:
            unique = np.unique(np.asarray(
                [int(destination) for destination in successors],
                dtype=np.int64))
        except (TypeError, ValueError) as error:
            raise DAGPreprocessingError(
                f"Invalid successor list for node {source}.") from error
        if unique.size and (unique[0] < 0 or unique[-1] >= node_count):
            bad = unique[0] if unique[0] < 0 else unique[-1]
            raise DAGPreprocessingError(
                f"DAG edge {source} -> {int(bad)} is out of bounds.")
        pieces.append(unique)
        dag_ptr[source + 1] = dag_ptr[source] + unique.size
    dag_index = (np.concatenate(pieces).astype(np.int32) if pieces
                 else np.zeros(0, dtype=np.int32))
    return dag_ptr, dag_index


def preprocess_sync_free(dag_successors, dep_count):
    dag_ptr, dag_index = compact_successors(dag_successors)
    dep_count = np.asarray(dep_count, dtype=np.int32)
    if dep_count.ndim != 1 or len(dep_count) != len(dag_successors):
        raise DAGPreprocessingError(
            "dep_count must contain one value for every DAG node.")
    if np.any(dep_count < 0):
        raise DAGPreprocessingError("Dependency counts cannot be negative.")
    return SyncFreeExecutionData(
        dep_count=dep_count.copy(), initial_dep_count=dep_count.copy(),
        dag_ptr=dag_ptr, dag_index=dag_index)


def wavefronts_from_dag(dag_successors, dep_count):
    """Level sets: the first holds every node without producers (ascending),
    each next one the ascending nodes released by the previous."""
    dag_ptr, dag_index = compact_successors(dag_successors)
    remaining = np.asarray(dep_count, dtype=np.int64).copy()
    wavefront = np.flatnonzero(remaining == 0)
    result = []
    while wavefront.size:
        result.append(wavefront.tolist())
        starts, ends = dag_ptr[wavefront], dag_ptr[wavefront + 1]
        total = int((ends - starts).sum())
        if total == 0:
            break
        offsets = np.repeat(starts - np.concatenate(
            ([0], np.cumsum(ends - starts)[:-1])), ends - starts)
        released = dag_index[np.arange(total) + offsets]
        np.subtract.at(remaining, released, 1)
        candidates = np.unique(released)
        wavefront = candidates[remaining[candidates] == 0]
    return result


def preprocess_wavefront(dag_successors, wavefront_list):
    node_count = len(dag_successors)
    wavefront_ptr = np.zeros(len(wavefront_list) + 1, dtype=np.int32)
    pieces = []
    seen = np.zeros(node_count, dtype=bool)
    for number, wavefront in enumerate(wavefront_list):
        try:
            nodes = np.asarray([int(node) for node in wavefront],
                               dtype=np.int64)
        except (TypeError, ValueError) as error:
            raise DAGPreprocessingError(
                f"Invalid node in wavefront {number}.") from error
        for node in nodes:
            if not 0 <= node < node_count:
                raise DAGPreprocessingError(
                    f"Wavefront node {int(node)} is out of bounds.")
            if seen[node]:
                raise DAGPreprocessingError(
                    f"DAG node {int(node)} occurs in more than one wavefront.")
            seen[node] = True
        pieces.append(nodes)
        wavefront_ptr[number + 1] = wavefront_ptr[number] + nodes.size
    if not seen.all():
        missing = np.flatnonzero(~seen).tolist()
        raise DAGPreprocessingError(
            "Wavefront scheduling did not cover every DAG node; the DAG may "
            f"contain a cycle. Missing nodes: {missing}.")
    wavefronts = (np.concatenate(pieces).astype(np.int32) if pieces
                  else np.zeros(0, dtype=np.int32))
    return WavefrontExecutionData(wavefronts=wavefronts,
                                  wavefront_ptr=wavefront_ptr)


def preprocess_warp_tasks(dag_successors, wavefront_list, band_width=1,
                          edge_count=None):
    if not isinstance(band_width, int) or band_width <= 0:
        raise DAGPreprocessingError(
            "The band width must be a positive integer.")
    node_count = len(dag_successors)
    dag_ptr, dag_index = compact_successors(dag_successors)
    wavefront_data = preprocess_wavefront(dag_successors, wavefront_list)
    nodes, level_ptr = wavefront_data.wavefronts, wavefront_data.wavefront_ptr
    if edge_count is None:
        dep_count = np.bincount(dag_index, minlength=node_count).astype(np.int32)
    else:
        dep_count = np.asarray(edge_count, dtype=np.int32)
        if dep_count.shape != (node_count,):
            raise DAGPreprocessingError(
                "edge_count must contain one value for every DAG node.")
    if band_width == 1:
        task_nodes = nodes
        task_ptr = np.arange(node_count + 1, dtype=np.int32)
        band_ptr = level_ptr.copy()
    else:
        task_nodes, task_ptr, band_ptr = band_chains(
            nodes, level_ptr, dag_ptr, dag_index, band_width)
    return WarpTaskExecutionData(
        task_nodes=task_nodes, task_ptr=task_ptr, band_ptr=band_ptr,
        dep_count=dep_count.copy(), initial_dep_count=dep_count.copy(),
        dag_ptr=dag_ptr, dag_index=dag_index)


def band_chains(nodes, level_ptr, dag_ptr, dag_index, band_width):
    """Connected components inside bands of ``band_width`` levels become
    sequential chain tasks (compiler/dag_preprocessing.py:258-298).
    Components are listed by first member, members keep band order."""
    level_count = len(level_ptr) - 1
    task_nodes, task_ptr, band_ptr = [], [0], [0]
    position_of = np.full(int(dag_ptr.size - 1), -1, dtype=np.int64)
    for first in range(0, level_count, band_width):
        last = min(first + band_width, level_count)
        band = np.asarray(nodes[level_ptr[first]:level_ptr[last]])
        position_of[band] = np.arange(band.size)
        parent = np.arange(band.size)

        def find(p):
            while parent[p] != p:
                parent[p] = parent[parent[p]]
                p = parent[p]
            return p

        for position, node in enumerate(band):
            for successor in dag_index[dag_ptr[node]:dag_ptr[node + 1]]:
                other = position_of[successor]
                if other >= 0:
                    a, b = find(position), find(other)
                    if a != b:
                        parent[b] = a
        chains = {}
        for position, node in enumerate(band):
            chains.setdefault(find(position), []).append(int(node))
        for chain in chains.values():
            task_nodes.extend(chain)
            task_ptr.append(len(task_nodes))
        band_ptr.append(len(task_ptr) - 1)
        position_of[band] = -1
    return (np.asarray(task_nodes, dtype=np.int32),
            np.asarray(task_ptr, dtype=np.int32),
            np.asarray(band_ptr, dtype=np.int32))


def execution_data_from_device_dag(dag, execution_mode, warp_mapped,
                                   pushed=False, band_width=1, mailbox=False,
                                   tile_rows=None, record_lanes=None,
                                   tile_boxes=None, level_positions=False):
    """Executor arrays straight from the on-device inspector (no host copy
    except the level offsets the launcher iterates over)."""
    if not isinstance(band_width, int) or band_width <= 0:
        raise DAGPreprocessingError(
            "The band width must be a positive integer.")
    if dag.scheduled != dag.n:
        raise DAGPreprocessingError(
            "Wavefront scheduling did not cover every DAG node; the DAG may "
            f"contain a cycle. Scheduled {dag.scheduled} of {dag.n} nodes.")
    counts = dag.array("edge_count" if pushed else "dep_count")
    if band_width != 1:
        # chain tasks: connected components inside bands of levels, built on
        # the device; only the band offsets come to the host (the launcher
        # iterates over them)
        if pushed or mailbox or tile_rows:
            raise DAGPreprocessingError(
                "band_width > 1 (chain tasks) runs on dependence counters.")
        dag.band_chains(band_width)
        return WarpTaskExecutionData(
            task_nodes=dag.array("task_nodes"), task_ptr=dag.array("task_ptr"),
            band_ptr=dag.host("band_ptr"), dep_count=counts,
            initial_dep_count=counts, dag_ptr=dag.array("dag_ptr"),
            dag_index=dag.array("dag_index"))
    task_nodes = dag.array("wavefronts")
    if level_positions and not tile_rows:
        # level launches over operands in level order: one tile that holds
        # every node is the level order itself, with its inverse beside it,
        # so the records can name a source by its place in that order
        task_nodes = dag.tile_order(max(int(dag.n), 1))
    if tile_rows:
        # tiled executor: tasks grouped by id // tile_rows, level order inside
        if not dag.topological_ids:
            raise DAGPreprocessingError(
                "The tiled executor needs every edge to go from a lower to a "
                "higher node id.")
        if tile_boxes is not None:
            # boxes of a structured grid; sources by their place in the queue
            grid, box = tile_boxes
            if not (mailbox and record_lanes) or (
                    int(np.prod(box)) != int(tile_rows)):
                raise DAGPreprocessingError(
                    "Box tiles need the mailbox protocol with task records "
                    "and tile_rows equal to the points of a box.")
            task_nodes = dag.box_order(grid, box)
        else:
            task_nodes = dag.tile_order(int(tile_rows))
    if mailbox:
        # destination v reads message slots in_ptr[v] .. in_ptr[v+1); the
        # entry at position p writes slot out_slot[p]; slot k carries the
        # product of position in_pos[k], made by task in_src[k]
        auxiliary = {"_lcd_in_ptr": dag.array("in_ptr"),
                     "_lcd_in_pos": dag.array("in_pos"),
                     "_lcd_in_src": dag.array("in_src"),
                     "_lcd_out_slot": dag.array("out_slot")}
        if record_lanes:
            # the first `record_lanes` incoming edges of every task, in the
            # order the executor visits the tasks
            records = dag.task_records(
                int(record_lanes),
                tiled=(2 if tile_boxes is not None or (
                    level_positions and not tile_rows) else bool(tile_rows)))
            auxiliary.update(zip(
                ("_lcd_rec_in", "_lcd_rec_src", "_lcd_rec_pos"), records))
        return WarpTaskExecutionData(
            task_nodes=task_nodes, task_ptr=None,
            band_ptr=dag.host("wavefront_ptr"), dep_count=counts,
            initial_dep_count=counts, dag_ptr=dag.array("dag_ptr"),
            dag_index=dag.array("dag_index"), auxiliary_values=auxiliary)
    if warp_mapped or execution_mode.replace("-", "_") == "sync_free":
        return WarpTaskExecutionData(
            task_nodes=task_nodes, task_ptr=None,
            band_ptr=dag.host("wavefront_ptr"), dep_count=counts,
            initial_dep_count=counts, dag_ptr=dag.array("dag_ptr"),
            dag_index=dag.array("dag_index"))
    return WavefrontExecutionData(
        wavefronts=dag.array("wavefronts"),
        wavefront_ptr=dag.host("wavefront_ptr"))

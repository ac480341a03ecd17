"""HIP runtime for generated `@parallel` kernels (ctypes over liblcdhip.so).

Counterpart of compiler/cuda_runtime.py of the reference: evaluates the
lifted host prelude, moves arrays to the device, compiles and binds the
generated module, runs the launcher, and restores the original return
semantics.  Device work goes through the C ABI declared in
``include/lcdhip.h``; there is no CPU execution path: without the library or a
GPU every entry point raises.

The *device layer* (``hip_module=`` parameters) is injectable like the
reference's ``cuda_module=``, so structural tests can substitute a fake.
"""

import ast
import ctypes
import hashlib
import os
import sys
from copy import deepcopy
from dataclasses import dataclass, field

import numpy as np

from lcd_amd.dag_preprocessing import (
    WarpTaskExecutionData,
    WavefrontExecutionData,
)

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(HERE, "liblcdhip.so")
HOST_LAUNCH_ARGUMENTS = frozenset({"wavefront_ptr", "band_ptr"})
STATUS_ARGUMENT = "_lcd_status"

(OK, ERR_HIP, ERR_COMPILE, ERR_ARGUMENT, ERR_DAG_BOUNDS, ERR_DAG_CYCLE,
 ERR_LOOKUP_POINTER, ERR_LOOKUP_ORDER, ERR_WATCHDOG, ERR_NO_DEVICE) = range(10)

DAG_PTR, DAG_INDEX, DAG_DEP_COUNT, DAG_EDGE_COUNT = 0, 1, 2, 3
DAG_LEVEL_OF, DAG_WAVEFRONTS, DAG_WAVEFRONT_PTR = 4, 5, 6
DAG_IN_PTR, DAG_IN_POS, DAG_OUT_SLOT, DAG_IN_SRC = 7, 8, 9, 10
DAG_TASK_NODES, DAG_TASK_PTR, DAG_BAND_PTR, DAG_TILE_NODES = 11, 12, 13, 14
DAG_REC_IN, DAG_REC_SRC, DAG_REC_POS, DAG_TILE_POS = 15, 16, 17, 18
# orders of lcdhip_dag_task_records
RECORDS_LEVEL_ORDER, RECORDS_TILE_ORDER, RECORDS_TILE_POSITIONS = 0, 1, 2
DAG_FLAG_LEVELS, DAG_FLAG_FORCE_KAHN, DAG_FLAG_INCOMING = 1, 2, 4

DEVICE_COMPILE_OPTIONS = (
    "--offload-arch=gfx950", "-O3", "-munsafe-fp-atomics",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


class HIPRuntimeError(Exception):
    """A liblcdhip call failed."""

    def __init__(self, message, code=ERR_HIP):
        super().__init__(message)
        self.code = code


class HIPRuntimePreparationError(Exception):
    """Lowered HIP arguments cannot be prepared."""


class HIPModuleCompilationError(Exception):
    """A generated HIP module cannot be compiled or bound."""


class ExecutorWatchdogError(HIPRuntimeError):
    """A sync-free executor gave up waiting (cyclic or corrupt schedule)."""


# --------------------------------------------------------------------------
# library binding

class _Props(ctypes.Structure):
    _fields_ = [
        ("compute_units", ctypes.c_int32), ("xcd_count", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("max_threads_per_block", ctypes.c_int32),
        ("lds_bytes_per_block", ctypes.c_int32),
        ("lds_bytes_per_cu", ctypes.c_int32), ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_bits", ctypes.c_int32), ("l2_bytes", ctypes.c_int32),
        ("global_memory_bytes", ctypes.c_int64),
        ("name", ctypes.c_char * 128), ("arch", ctypes.c_char * 64),
    ]


class _Arch(ctypes.Structure):
    _fields_ = [(name, ctypes.c_double) for name in (
        "launch_latency_s", "atomic_cost_s", "memory_bandwidth_bytes_per_s",
        "lane_flops_per_s", "handoff_s", "barrier_s", "graph_node_s",
        "lds_handoff_s", "chain_step_s")]


RULE_SEGMENT, RULE_LATER, RULE_NEXT = 0, 1, 2


class _DagRule(ctypes.Structure):
    _fields_ = [
        ("d_ptr", ctypes.c_void_p), ("d_idx", ctypes.c_void_p),
        ("idx_size", ctypes.c_int64), ("owner_is_source", ctypes.c_int32),
        ("lower_offset", ctypes.c_int32), ("upper_offset", ctypes.c_int32),
        ("guard", ctypes.c_int32), ("break_at_owner", ctypes.c_int32),
        ("relation", ctypes.c_int32),
    ]


class _DagInfo(ctypes.Structure):
    _fields_ = [
        ("n", ctypes.c_int64), ("edges", ctypes.c_int64),
        ("levels", ctypes.c_int64), ("scheduled", ctypes.c_int64),
        ("max_level_width", ctypes.c_int64),
        ("topological_ids", ctypes.c_int32),
        ("level_algorithm", ctypes.c_int32),
    ]


EXPORTED_SYMBOLS = (
    "lcdhip_last_error", "lcdhip_version", "lcdhip_init", "lcdhip_shutdown",
    "lcdhip_device_count", "lcdhip_device_props", "lcdhip_measure_arch",
    "lcdhip_buffer_alloc", "lcdhip_buffer_free", "lcdhip_buffer_upload",
    "lcdhip_buffer_download", "lcdhip_buffer_copy", "lcdhip_buffer_fill32",
    "lcdhip_host_alloc", "lcdhip_host_free", "lcdhip_stream_create",
    "lcdhip_stream_destroy", "lcdhip_stream_sync", "lcdhip_event_create",
    "lcdhip_event_destroy", "lcdhip_event_record", "lcdhip_event_elapsed_ms",
    "lcdhip_module_compile_code", "lcdhip_free_host", "lcdhip_module_load",
    "lcdhip_module_destroy", "lcdhip_module_get_kernel",
    "lcdhip_kernel_max_resident_blocks", "lcdhip_launch",
    "lcdhip_launch_levels", "lcdhip_graph_begin_capture",
    "lcdhip_graph_end_capture", "lcdhip_graph_launch", "lcdhip_graph_destroy",
    "lcdhip_dag_build", "lcdhip_dag_get_info", "lcdhip_dag_array",
    "lcdhip_dag_download", "lcdhip_dag_destroy", "lcdhip_dag_band_chains",
    "lcdhip_dag_tile_order", "lcdhip_dag_tile_locality",
    "lcdhip_dag_box_order", "lcdhip_dag_edge_offsets",
    "lcdhip_pair_lookup_build",
    "lcdhip_pair_offsets_build",
    "lcdhip_dag_task_records",
    "lcdhip_lookup_build", "lcdhip_gather_i32",
    "lcdhip_digest", "lcdhip_digest_noalloc",
)

_library = None


def load_library():
    """Load ``liblcdhip.so``; raise if it has not been built."""
    global _library
    if _library is not None:
        return _library
    if not os.path.exists(LIBRARY_PATH):
        raise HIPRuntimeError(
            f"{LIBRARY_PATH} is missing: build it with `python -m "
            "lcd_amd.build` (hipcc, gfx950). There is no CPU fallback.",
            ERR_NO_DEVICE)
    lib = ctypes.CDLL(LIBRARY_PATH)
    lib.lcdhip_last_error.restype = ctypes.c_char_p
    lib.lcdhip_version.restype = ctypes.c_char_p
    for name in EXPORTED_SYMBOLS:
        function = getattr(lib, name)
        if name not in ("lcdhip_last_error", "lcdhip_version",
                        "lcdhip_free_host"):
            function.restype = ctypes.c_int
    lib.lcdhip_free_host.restype = None
    lib.lcdhip_free_host.argtypes = [ctypes.c_void_p]
    _library = lib
    return lib


def _check(status):
    if status != OK:
        message = load_library().lcdhip_last_error().decode(errors="replace")
        if status == ERR_WATCHDOG:
            raise ExecutorWatchdogError(message, status)
        raise HIPRuntimeError(message, status)


_hook_notices = set()


def _warn_hook(variable, what):
    """One warning per process and developer hook that takes effect: the
    kernels that run are then not the ones this package generates."""
    if variable in _hook_notices:
        return
    _hook_notices.add(variable)
    import warnings
    warnings.warn(f"lcd_amd: {variable} is set: {what}", RuntimeWarning,
                  stacklevel=3)


def code_cache_directory():
    """Where compiled code objects are kept between processes, or None when
    the cache is switched off (``LCD_HIP_CACHE=0``): ``LCD_HIP_CACHE_DIR``,
    else ``$XDG_CACHE_HOME/lcd_amd/hiprtc`` (``~/.cache`` by default)."""
    if os.environ.get("LCD_HIP_CACHE", "1").strip().lower() in (
            "0", "off", "no", "false"):
        return None
    chosen = os.environ.get("LCD_HIP_CACHE_DIR")
    if chosen:
        return chosen
    base = os.environ.get("XDG_CACHE_HOME") or os.path.join(
        os.path.expanduser("~"), ".cache")
    return os.path.join(base, "lcd_amd", "hiprtc")


_CACHE_MAGIC = b"LCDHIPCO1\n"


def _cache_path(lib, source, opts):
    directory = code_cache_directory()
    if directory is None:
        return None
    key = hashlib.sha256()
    for part in (lib.lcdhip_version(), b"\0".join(opts), source.encode()):
        key.update(len(part).to_bytes(8, "little"))
        key.update(part)
    return os.path.join(directory, key.hexdigest() + ".co")


def _cache_read(path):
    """The code object kept under ``path``, or None: no such entry, or one
    that is not whole (the payload carries its own SHA-256)."""
    try:
        with open(path, "rb") as handle:
            blob = handle.read()
    except OSError:
        return None
    head = len(_CACHE_MAGIC)
    if len(blob) < head + 32 or blob[:head] != _CACHE_MAGIC:
        return None
    digest, code = blob[head:head + 32], blob[head + 32:]
    if hashlib.sha256(code).digest() != digest or not code:
        return None
    return code


def _cache_write(path, code):
    """Atomically (write beside, rename); a cache that cannot be written is
    no error."""
    try:
        os.makedirs(os.path.dirname(path), exist_ok=True)
        temporary = f"{path}.{os.getpid()}.tmp"
        with open(temporary, "wb") as handle:
            handle.write(_CACHE_MAGIC + hashlib.sha256(code).digest() + code)
        os.replace(temporary, path)
    except OSError:
        pass


code_cache_statistics = {"hits": 0, "misses": 0}


def compile_code(source, name="lcd_generated.hip", options=()):
    """hiprtc-compile HIP source for gfx950; works without a GPU.

    The code object is kept on disk under a key of the source text, every
    option, the target and the versions of this library and of hiprtc, and
    loaded from there by the next process (the reference keeps its compiled
    variants for the life of one process, compiler/decorator.py:201-245;
    hiprtc takes 0.1-0.3 s per kernel).  ``code_cache_directory`` says where
    and how to switch it off."""
    lib = load_library()
    extra = tuple(os.environ.get("LCD_HIP_EXTRA_OPTIONS", "").split())
    if extra:
        _warn_hook("LCD_HIP_EXTRA_OPTIONS",
                   f"every kernel is compiled with the extra options {extra}.")
    opts = [o.encode() for o in (*DEVICE_COMPILE_OPTIONS, *options, *extra)]
    cached = _cache_path(lib, source, opts)
    if cached is not None:
        data = _cache_read(cached)
        if data is not None:
            code_cache_statistics["hits"] += 1
            return data, ""
    code_cache_statistics["misses"] += 1
    array = (ctypes.c_char_p * len(opts))(*opts)
    code, size, log = ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_char_p()
    status = lib.lcdhip_module_compile_code(
        source.encode(), name.encode(), array, len(opts), ctypes.byref(code),
        ctypes.byref(size), ctypes.byref(log))
    log_text = log.value.decode(errors="replace") if log.value else ""
    if log:
        lib.lcdhip_free_host(log)
    if status != OK:
        message = lib.lcdhip_last_error().decode(errors="replace")
        raise HIPModuleCompilationError(
            f"Failed to compile the generated HIP module {name}:\n{message}")
    data = ctypes.string_at(code, size.value)
    lib.lcdhip_free_host(code)
    if cached is not None:
        _cache_write(cached, data)
    return data, log_text


# --------------------------------------------------------------------------
# device objects

_CTYPES = {"int": ctypes.c_int32, "long long": ctypes.c_int64,
           "double": ctypes.c_double, "float": ctypes.c_float}
_DTYPE_TO_C = {"int8": "signed char", "int32": "int", "int64": "long long",
               "float64": "double",
               "float32": "float", "uint32": "unsigned int",
               "uint64": "unsigned long long"}


class DeviceArray:
    """A 1-D (or flat n-D) array in HBM owned by this process."""

    def __init__(self, device, pointer, shape, dtype, owner=True, base=None):
        self.device = device
        self.pointer = int(pointer)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.owner = owner
        self._base = base

    @property
    def size(self):
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def nbytes(self):
        return self.size * self.dtype.itemsize

    def __len__(self):
        return self.shape[0] if self.shape else 1

    @property
    def __cuda_array_interface__(self):
        return {"shape": self.shape, "typestr": self.dtype.str,
                "data": (self.pointer, False), "version": 3, "strides": None}

    def copy_to_host(self, out=None):
        if out is None:
            out = np.empty(self.shape, dtype=self.dtype)
        self.device.download(out, self)
        return out

    def free(self):
        if self.owner and self.pointer:
            _check(load_library().lcdhip_buffer_free(
                ctypes.c_void_p(self.pointer)))
        self.pointer = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def is_device_array(value):
    return hasattr(value, "__cuda_array_interface__")


def device_pointer(value):
    if isinstance(value, DeviceArray):
        return value.pointer
    return int(value.__cuda_array_interface__["data"][0])


def device_array_meta(value):
    if isinstance(value, DeviceArray):
        return value.shape, value.dtype
    interface = value.__cuda_array_interface__
    return tuple(interface["shape"]), np.dtype(interface["typestr"])


class HIPKernel:
    def __init__(self, handle, name, argument_ctypes):
        self.handle = handle
        self.name = name
        self.argument_ctypes = argument_ctypes


class HIPModule:
    """One loaded code object and its kernels."""

    def __init__(self, device, code, argument_ctypes):
        self.device = device
        self.argument_ctypes = argument_ctypes   # kernel name -> [ctypes]
        handle = ctypes.c_void_p()
        _check(load_library().lcdhip_module_load(
            code, ctypes.c_size_t(len(code)), ctypes.byref(handle)))
        self.handle = handle
        self._kernels = {}

    def kernel(self, name):
        if name not in self._kernels:
            handle = ctypes.c_void_p()
            status = load_library().lcdhip_module_get_kernel(
                self.handle, name.encode(), ctypes.byref(handle))
            if status != OK:
                raise HIPModuleCompilationError(
                    f"Generated HIP symbol {name!r} was not bound.")
            self._kernels[name] = HIPKernel(
                handle, name, self.argument_ctypes.get(name))
        return self._kernels[name]


class HIPGraph:
    def __init__(self, device, handle):
        self.device = device
        self.handle = handle

    def launch(self, stream=None):
        _check(load_library().lcdhip_graph_launch(self.handle, stream))

    def destroy(self):
        if self.handle:
            load_library().lcdhip_graph_destroy(self.handle)
            self.handle = None


class DeviceDag:
    """Handle of one on-device DAG (edges, counts, level sets)."""

    ARRAYS = {"dag_ptr": DAG_PTR, "dag_index": DAG_INDEX,
              "dep_count": DAG_DEP_COUNT, "edge_count": DAG_EDGE_COUNT,
              "level_of": DAG_LEVEL_OF, "wavefronts": DAG_WAVEFRONTS,
              "wavefront_ptr": DAG_WAVEFRONT_PTR, "in_ptr": DAG_IN_PTR,
              "in_pos": DAG_IN_POS, "out_slot": DAG_OUT_SLOT,
              "in_src": DAG_IN_SRC, "task_nodes": DAG_TASK_NODES,
              "task_ptr": DAG_TASK_PTR, "band_ptr": DAG_BAND_PTR,
              "tile_nodes": DAG_TILE_NODES, "rec_in": DAG_REC_IN,
              "rec_src": DAG_REC_SRC, "rec_pos": DAG_REC_POS,
              "tile_pos": DAG_TILE_POS}
    CHAIN_ARRAYS = ("task_nodes", "task_ptr", "band_ptr")

    def __init__(self, device, handle):
        self.device = device
        self.handle = handle
        info = _DagInfo()
        _check(load_library().lcdhip_dag_get_info(handle, ctypes.byref(info)))
        self.n, self.edges = int(info.n), int(info.edges)
        self.levels, self.scheduled = int(info.levels), int(info.scheduled)
        self.max_level_width = int(info.max_level_width)
        self.topological_ids = bool(info.topological_ids)
        self.level_algorithm = int(info.level_algorithm)
        self._views = {}
        self._host = {}

    def array(self, name):
        """Device view (not owned) of one DAG array."""
        if name not in self._views:
            pointer, count = ctypes.c_void_p(), ctypes.c_int64()
            _check(load_library().lcdhip_dag_array(
                self.handle, self.ARRAYS[name], ctypes.byref(pointer),
                ctypes.byref(count)))
            self._views[name] = DeviceArray(
                self.device, pointer.value or 0, (count.value,), np.int32,
                owner=False, base=self)
        return self._views[name]

    def host(self, name):
        if name not in self._host:
            view = self.array(name)
            out = np.empty(view.shape, dtype=np.int32)
            _check(load_library().lcdhip_dag_download(
                self.handle, self.ARRAYS[name],
                out.ctypes.data_as(ctypes.c_void_p), ctypes.c_int64(out.size)))
            self._host[name] = out
        return self._host[name]

    def band_chains(self, band_width):
        """Build the chain tasks of bands of ``band_width`` levels on the
        device; afterwards ``task_nodes``, ``task_ptr`` and ``band_ptr`` are
        arrays of this DAG.  Returns ``(tasks, bands)``."""
        if not isinstance(band_width, int) or band_width <= 0:
            raise HIPRuntimeError("The band width must be a positive integer.",
                                  ERR_ARGUMENT)
        for name in self.CHAIN_ARRAYS:
            self._views.pop(name, None)
            self._host.pop(name, None)
        tasks, bands = ctypes.c_int64(), ctypes.c_int64()
        _check(load_library().lcdhip_dag_band_chains(
            self.handle, ctypes.c_int64(band_width), self.device.stream,
            ctypes.byref(tasks), ctypes.byref(bands)))
        self.chain_band_width = band_width
        return int(tasks.value), int(bands.value)

    def tile_locality(self, tile_rows):
        """Share of the edges whose endpoints share a tile of ``tile_rows``
        consecutive ids."""
        if self.edges == 0:
            return 1.0
        local = ctypes.c_int64()
        _check(load_library().lcdhip_dag_tile_locality(
            self.handle, ctypes.c_int64(int(tile_rows)), self.device.stream,
            ctypes.byref(local)))
        return local.value / self.edges

    def tile_order(self, tile_rows):
        """Order the nodes by (id // tile_rows, level, id) on the device;
        afterwards ``tile_nodes`` is an array of this DAG."""
        if not isinstance(tile_rows, int) or tile_rows <= 0:
            raise HIPRuntimeError("The tile size must be a positive integer.",
                                  ERR_ARGUMENT)
        for name in ("tile_nodes", "tile_pos"):
            self._views.pop(name, None)
            self._host.pop(name, None)
        _check(load_library().lcdhip_dag_tile_order(
            self.handle, ctypes.c_int64(tile_rows), self.device.stream))
        self.tile_rows = tile_rows
        return self.array("tile_nodes")

    def box_order(self, grid, box):
        """Order the nodes of a structured grid (id = x + nx * (y + ny * z))
        by (box, level, id), boxes of ``box`` grid points in (z, y, x) order;
        afterwards ``tile_nodes`` and ``tile_pos`` (its inverse) are arrays
        of this DAG."""
        grid, box = tuple(grid), tuple(box)
        if len(grid) != 3 or len(box) != 3 or not all(
                isinstance(extent, (int, np.integer)) and extent > 0
                for extent in grid + box):
            raise HIPRuntimeError(
                "Grid and box are three positive integers each.", ERR_ARGUMENT)
        for name in ("tile_nodes", "tile_pos"):
            self._views.pop(name, None)
            self._host.pop(name, None)
        extents = ctypes.c_int64 * 3
        _check(load_library().lcdhip_dag_box_order(
            self.handle, extents(*map(int, grid)), extents(*map(int, box)),
            self.device.stream))
        self.tile_rows = int(box[0]) * int(box[1]) * int(box[2])
        return self.array("tile_nodes")

    def edge_offsets(self, capacity=16):
        """``(offsets, counts, distinct)``: the distinct values of
        destination - source over the edges (the first ``capacity`` of them,
        ascending), how many edges have each, and how many values there
        are."""
        offsets = (ctypes.c_int64 * max(capacity, 1))()
        counts = (ctypes.c_int64 * max(capacity, 1))()
        distinct = ctypes.c_int64()
        _check(load_library().lcdhip_dag_edge_offsets(
            self.handle, ctypes.c_int64(capacity), offsets, counts,
            ctypes.byref(distinct), self.device.stream))
        take = min(capacity, distinct.value)
        return (list(offsets[:take]), list(counts[:take]),
                int(distinct.value))

    def task_records(self, lanes, tiled=False):
        """Fixed-size records of the incoming listing in task order
        (``tile_nodes`` when ``tiled``, else ``wavefronts``):
        afterwards ``rec_in`` (2 per task), ``rec_src`` and ``rec_pos``
        (``lanes`` per task) are arrays of this DAG.  ``tiled`` may be
        ``RECORDS_TILE_POSITIONS``: sources are then named by their position
        in ``tile_nodes``, and an order that is not topological is an
        error."""
        if not isinstance(lanes, int) or not 1 <= lanes <= 64:
            raise HIPRuntimeError(
                "Task records need 1 to 64 lanes per task.", ERR_ARGUMENT)
        for name in ("rec_in", "rec_src", "rec_pos"):
            self._views.pop(name, None)
            self._host.pop(name, None)
        overflow = ctypes.c_int64()
        _check(load_library().lcdhip_dag_task_records(
            self.handle, ctypes.c_int(lanes),
            ctypes.c_int(int(tiled)),   # False / True / RECORDS_*
            self.device.stream, ctypes.byref(overflow)))
        self.record_lanes = lanes
        # tasks whose incoming edges do not all fit their record
        self.record_overflow = int(overflow.value)
        return tuple(self.array(name)
                     for name in ("rec_in", "rec_src", "rec_pos"))

    def successors(self):
        ptr, index = self.host("dag_ptr"), self.host("dag_index")
        return [index[ptr[v]:ptr[v + 1]].tolist() for v in range(self.n)]

    def wavefront_list(self):
        ptr, nodes = self.host("wavefront_ptr"), self.host("wavefronts")
        return [nodes[ptr[k]:ptr[k + 1]].tolist() for k in range(self.levels)]

    def destroy(self):
        if self.handle:
            load_library().lcdhip_dag_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class HIPDevice:
    """One GPU context: the default device layer of the runtime."""

    def __init__(self, index=0):
        self.lib = load_library()
        _check(self.lib.lcdhip_init(index))
        self.index = index
        self._props = None
        self._arch = None
        self.stream = None   # None = the library's default stream

    # ---- properties
    @property
    def props(self):
        if self._props is None:
            props = _Props()
            _check(self.lib.lcdhip_device_props(ctypes.byref(props)))
            self._props = props
        return self._props

    def measure_arch(self):
        if self._arch is None:
            arch = _Arch()
            _check(self.lib.lcdhip_measure_arch(ctypes.byref(arch)))
            self._arch = {name: getattr(arch, name) for name, _ in _Arch._fields_}
        return dict(self._arch)

    # ---- memory
    def empty(self, shape, dtype):
        shape = (shape,) if np.isscalar(shape) else tuple(shape)
        dtype = np.dtype(dtype)
        pointer = ctypes.c_void_p()
        nbytes = int(np.prod(shape)) * dtype.itemsize
        _check(self.lib.lcdhip_buffer_alloc(ctypes.c_size_t(nbytes),
                                            ctypes.byref(pointer)))
        return DeviceArray(self, pointer.value, shape, dtype)

    def zeros(self, shape, dtype=np.float64):
        array = self.empty(shape, dtype)
        self.fill_zero(array)
        return array

    def fill_zero(self, array):
        if array.nbytes % 4:
            raise HIPRuntimePreparationError("fill needs 4-byte multiples")
        _check(self.lib.lcdhip_buffer_fill32(
            ctypes.c_void_p(array.pointer), ctypes.c_uint32(0),
            ctypes.c_size_t(array.nbytes // 4), self.stream))

    def to_device(self, value, into=None):
        value = np.ascontiguousarray(value)
        if into is None or into.nbytes != value.nbytes or (
                into.dtype != value.dtype):
            into = self.empty(value.shape, value.dtype)
        _check(self.lib.lcdhip_buffer_upload(
            ctypes.c_void_p(into.pointer),
            value.ctypes.data_as(ctypes.c_void_p),
            ctypes.c_size_t(value.nbytes), self.stream))
        # pageable source: the copy has consumed the host buffer only after a
        # synchronise
        self.synchronize()
        return into

    def download(self, out, array):
        _check(self.lib.lcdhip_buffer_download(
            out.ctypes.data_as(ctypes.c_void_p),
            ctypes.c_void_p(device_pointer(array)),
            ctypes.c_size_t(out.nbytes), self.stream))
        self.synchronize()

    def copy(self, destination, source):
        _check(self.lib.lcdhip_buffer_copy(
            ctypes.c_void_p(device_pointer(destination)),
            ctypes.c_void_p(device_pointer(source)),
            ctypes.c_size_t(destination.nbytes), self.stream))

    def synchronize(self):
        _check(self.lib.lcdhip_stream_sync(self.stream))

    # ---- events
    def event(self):
        handle = ctypes.c_void_p()
        _check(self.lib.lcdhip_event_create(ctypes.byref(handle)))
        return handle

    def record(self, event):
        _check(self.lib.lcdhip_event_record(event, self.stream))

    def elapsed_ms(self, start, stop):
        ms = ctypes.c_float()
        _check(self.lib.lcdhip_event_elapsed_ms(start, stop, ctypes.byref(ms)))
        return float(ms.value)

    # ---- modules and launches
    def load_module(self, code, argument_ctypes):
        return HIPModule(self, code, argument_ctypes)

    def resident_blocks(self, kernel, block):
        blocks = ctypes.c_int()
        _check(self.lib.lcdhip_kernel_max_resident_blocks(
            kernel.handle, int(block), ctypes.c_size_t(0),
            ctypes.byref(blocks)))
        return int(blocks.value)

    @staticmethod
    def _marshal(kernel, args):
        types = kernel.argument_ctypes
        if types is None or len(types) != len(args):
            raise HIPRuntimePreparationError(
                f"Kernel {kernel.name} expects "
                f"{None if types is None else len(types)} arguments, got "
                f"{len(args)}.")
        holders = []
        for ctype, value in zip(types, args):
            if ctype is ctypes.c_void_p:
                if value is None:
                    holders.append(ctypes.c_void_p(0))
                elif is_device_array(value):
                    holders.append(ctypes.c_void_p(device_pointer(value)))
                else:
                    raise HIPRuntimePreparationError(
                        f"Kernel {kernel.name}: expected a device array, got "
                        f"{type(value).__name__}.")
            else:
                holders.append(ctype(value))
        pointers = (ctypes.c_void_p * len(holders))(
            *[ctypes.cast(ctypes.pointer(h), ctypes.c_void_p) for h in holders])
        return holders, pointers

    def launch(self, kernel, grid, block, args):
        holders, pointers = self._marshal(kernel, args)
        _check(self.lib.lcdhip_launch(
            kernel.handle, ctypes.c_uint32(int(grid)),
            ctypes.c_uint32(int(block)), ctypes.c_size_t(0), self.stream,
            pointers))

    def launch_levels(self, kernel, host_ptr, tasks_per_block, block, args,
                      start_index, end_index):
        host_ptr = np.ascontiguousarray(host_ptr, dtype=np.int32)
        holders, pointers = self._marshal(kernel, args)
        _check(self.lib.lcdhip_launch_levels(
            kernel.handle, host_ptr.ctypes.data_as(ctypes.c_void_p),
            ctypes.c_int64(len(host_ptr) - 1), ctypes.c_int32(tasks_per_block),
            ctypes.c_uint32(int(block)), ctypes.c_size_t(0), self.stream,
            pointers, int(start_index), int(end_index)))

    def begin_capture(self):
        _check(self.lib.lcdhip_graph_begin_capture(self.stream))

    def end_capture(self):
        handle = ctypes.c_void_p()
        _check(self.lib.lcdhip_graph_end_capture(self.stream,
                                                 ctypes.byref(handle)))
        return HIPGraph(self, handle)

    # ---- inspector
    def _resident_int32(self, value, keep):
        if is_device_array(value):
            shape, dtype = device_array_meta(value)
            if dtype != np.int32:
                raise HIPRuntimePreparationError(
                    "structure arrays must be int32 on the device")
            return device_pointer(value), int(np.prod(shape))
        host = np.ascontiguousarray(value)
        if not np.issubdtype(host.dtype, np.integer):
            raise HIPRuntimePreparationError(
                "structure arrays must hold integers")
        array = self.to_device(host.astype(np.int32, copy=False))
        keep.append(array)
        return array.pointer, array.size

    def dag_build(self, rules, n, levels=True, force_kahn=False,
                  incoming=False):
        """Run the on-device inspector. ``rules`` are dicts/objects with
        ptr, idx, owner_is_source, lower_offset, upper_offset, guard,
        break_at_owner (ptr/idx host or device arrays), or, for the
        relational rule ``seg -> every j >= seg + lower_offset``, with
        ``relation=RULE_LATER`` and ``lower_offset`` only (``RULE_NEXT``: the
        single edge ``seg -> seg + lower_offset``)."""
        keep = []
        array = (_DagRule * max(len(rules), 1))()
        for slot, rule in zip(array, rules):
            get = rule.get if isinstance(rule, dict) else (
                lambda key, r=rule: getattr(r, key, None))
            if int(get("relation") or 0) in (RULE_LATER, RULE_NEXT):
                slot.relation = int(get("relation"))
                slot.lower_offset = int(get("lower_offset"))
                continue
            slot.d_ptr, _ = self._resident_int32(get("ptr"), keep)
            slot.d_idx, slot.idx_size = self._resident_int32(get("idx"), keep)
            slot.owner_is_source = int(bool(get("owner_is_source")))
            slot.lower_offset = int(get("lower_offset"))
            slot.upper_offset = int(get("upper_offset"))
            slot.guard = int(get("guard"))
            slot.break_at_owner = int(bool(get("break_at_owner")))
        flags = (DAG_FLAG_LEVELS if levels else 0) | (
            DAG_FLAG_FORCE_KAHN if force_kahn else 0) | (
            DAG_FLAG_INCOMING if incoming else 0)
        handle = ctypes.c_void_p()
        _check(self.lib.lcdhip_dag_build(
            array, len(rules), ctypes.c_int64(int(n)), ctypes.c_uint32(flags),
            self.stream, ctypes.byref(handle)))
        return DeviceDag(self, handle)

    def lookup_build(self, pointers, indices):
        keep = []
        d_ptr, ptr_size = self._resident_int32(pointers, keep)
        d_idx, idx_size = self._resident_int32(indices, keep)
        n = ptr_size - 1
        out = self.empty((max(n, 0),), np.int32)
        _check(self.lib.lcdhip_lookup_build(
            ctypes.c_void_p(d_ptr), ctypes.c_void_p(d_idx), ctypes.c_int64(n),
            ctypes.c_int64(idx_size), ctypes.c_void_p(out.pointer),
            self.stream))
        return out

    def pair_lookup_entries(self, pointers, indices):
        """Entries a pair table of this structure would have (the sum of the
        squared segment lengths)."""
        keep = []
        d_ptr, ptr_size = self._resident_int32(pointers, keep)
        d_idx, idx_size = self._resident_int32(indices, keep)
        entries = ctypes.c_int64()
        _check(self.lib.lcdhip_pair_lookup_build(
            ctypes.c_void_p(d_ptr), ctypes.c_void_p(d_idx),
            ctypes.c_int64(ptr_size - 1), ctypes.c_int64(idx_size), None, None,
            ctypes.c_int64(0), ctypes.byref(entries), self.stream))
        return int(entries.value)

    def pair_lookup_build(self, pointers, indices, offsets=False):
        """``(base, table)``: for segment s with entries a, b,
        ``table[base[s] + a * len + b]`` is the position in segment
        ``indices[pointers[s] + a]`` of the index ``indices[pointers[s] +
        b]``, or -1.  With ``offsets`` the table holds one byte per entry:
        the position's offset from the start of the segment searched
        (segments of at most 127 entries)."""
        keep = []
        d_ptr, ptr_size = self._resident_int32(pointers, keep)
        d_idx, idx_size = self._resident_int32(indices, keep)
        n = ptr_size - 1
        entries = self.pair_lookup_entries(pointers, indices)
        base = self.empty((n + 1,), np.int32)
        table = self.empty((max(entries, 1),),
                           np.int8 if offsets else np.int32)
        build = (self.lib.lcdhip_pair_offsets_build if offsets
                 else self.lib.lcdhip_pair_lookup_build)
        _check(build(
            ctypes.c_void_p(d_ptr), ctypes.c_void_p(d_idx), ctypes.c_int64(n),
            ctypes.c_int64(idx_size), ctypes.c_void_p(base.pointer),
            ctypes.c_void_p(table.pointer), ctypes.c_int64(entries),
            ctypes.byref(entries_out := ctypes.c_int64()), self.stream))
        return base, table

    def gather_int32(self, source, index, offset=0):
        """``source[index[q] + offset]`` for every ``q``, on the device."""
        keep = []
        d_src, src_size = self._resident_int32(source, keep)
        d_index, count = self._resident_int32(index, keep)
        out = self.empty((max(count, 0),), np.int32)
        _check(self.lib.lcdhip_gather_i32(
            ctypes.c_void_p(out.pointer), ctypes.c_void_p(d_src),
            ctypes.c_void_p(d_index), ctypes.c_int64(int(offset)),
            ctypes.c_int64(count), ctypes.c_int64(src_size), self.stream))
        return out

    def digest(self, array):
        out = (ctypes.c_uint64 * 2)()
        shape, dtype = device_array_meta(array)
        nbytes = int(np.prod(shape)) * dtype.itemsize
        _check(self.lib.lcdhip_digest(
            ctypes.c_void_p(device_pointer(array)), ctypes.c_size_t(nbytes),
            out, self.stream))
        return int(out[0]), int(out[1])

    def digest_noalloc(self, array, out):
        """Enqueue the digest of ``array`` into the device array ``out``
        (two uint64) without allocating or synchronising
        (``lcdhip_digest_noalloc``)."""
        shape, dtype = device_array_meta(array)
        nbytes = int(np.prod(shape)) * dtype.itemsize
        out_shape, out_dtype = device_array_meta(out)
        if int(np.prod(out_shape)) * out_dtype.itemsize < 16:
            raise HIPRuntimePreparationError(
                "digest_noalloc needs 16 bytes of device memory for the result")
        _check(self.lib.lcdhip_digest_noalloc(
            ctypes.c_void_p(device_pointer(array)), ctypes.c_size_t(nbytes),
            ctypes.c_void_p(device_pointer(out)), self.stream))


_default_device = None


def default_device():
    """The process-wide GPU context (device 0); raises without a GPU."""
    global _default_device
    if _default_device is None:
        _default_device = HIPDevice(0)
    return _default_device


def device_available():
    try:
        count = ctypes.c_int()
        status = load_library().lcdhip_device_count(ctypes.byref(count))
        return status == OK and count.value > 0
    except (HIPRuntimeError, OSError):
        return False


# --------------------------------------------------------------------------
# compile / prepare / execute (the reference's cuda_runtime entry points)

@dataclass
class CompiledHIPModule:
    """Compiled code objects and the Python launcher of one lowering."""

    lowering: object
    launcher: object
    namespace: dict
    kernel: object = None            # kernel name (bound lazily per device)
    code_objects: dict = field(default_factory=dict)   # type key -> bytes
    loaded: dict = field(default_factory=dict)         # (device, key) -> HIPModule

    def type_options(self, array_types, scalar_types):
        options = []
        for name in self.lowering.kernel_arguments:
            if name in array_types:
                options.append(f"-DLCD_T_{name}={array_types[name]}")
            elif name in scalar_types:
                options.append(f"-DLCD_T_{name}={scalar_types[name]}")
        return tuple(options)

    def code_for(self, options=()):
        key = tuple(options)
        if key not in self.code_objects:
            source = self.lowering.source
            # developer aids: LCD_HIP_DUMP_DIR writes every generated module,
            # LCD_HIP_OVERRIDE_DIR/<kernel>.hip replaces one with edited text
            dump = os.environ.get("LCD_HIP_DUMP_DIR")
            if dump:
                os.makedirs(dump, exist_ok=True)
                with open(os.path.join(
                        dump, self.lowering.kernel_name + ".hip"), "w") as out:
                    out.write(source)
            override = os.environ.get("LCD_HIP_OVERRIDE_DIR")
            if override:
                path = os.path.join(override, self.lowering.kernel_name + ".hip")
                if os.path.exists(path):
                    _warn_hook("LCD_HIP_OVERRIDE_DIR",
                               f"the text of {path} replaces the generated "
                               f"kernel {self.lowering.kernel_name}.")
                    with open(path) as handle:
                        source = handle.read()
            digest = hashlib.blake2b(
                (source + "\0".join(key)).encode(),
                digest_size=8).hexdigest()
            code, _ = compile_code(
                source, f"{self.lowering.function_name}_{digest}.hip", key)
            self.code_objects[key] = code
        return self.code_objects[key]


def _default_types(lowering):
    arrays = {name: ("int" if kind == "int" else "double")
              for name, kind in lowering.array_arguments.items()}
    scalars = {}
    for name, kind in lowering.scalar_arguments.items():
        if name in ("band_start", "band_end", "task_count"):
            scalars[name] = "int"
        else:
            scalars[name] = "long long" if kind == "int" else "double"
    return arrays, scalars


def compile_hip_module(lowering, function_globals=None, hip_module=None,
                       precompile=True):
    """Bind the generated launcher and compile the generated HIP source.

    Mirrors ``compile_cuda_module`` (compiler/cuda_runtime.py:70-125).  The
    device code is compiled by hiprtc for the default argument types right
    away (this needs no GPU and surfaces compiler diagnostics at decoration
    time); a differently typed call compiles its own specialisation.
    """
    namespace = dict(function_globals or {})
    try:
        exec(compile(lowering.launcher_ast, "<generated-hip-launcher>", "exec"),
             namespace, namespace)
        launcher = namespace[lowering.launcher_name]
    except Exception as error:
        raise HIPModuleCompilationError(
            "Failed to bind the generated HIP launcher.") from error
    if not callable(launcher):
        raise HIPModuleCompilationError(
            "The generated HIP launcher must be callable.")
    compiled = CompiledHIPModule(
        lowering=lowering, launcher=launcher, namespace=namespace,
        kernel=lowering.kernel_name)
    namespace["hip"] = hip_module
    if precompile and hip_module is None:
        compiled.code_for(())
    return compiled


class LaunchContext:
    """The ``_hip`` object the generated launcher drives."""

    def __init__(self, device, module, lengths):
        self.device = device
        self.module = module
        self.lengths = lengths

    def length(self, array):
        if isinstance(array, DeviceArray) or is_device_array(array):
            return int(device_array_meta(array)[0][0])
        return len(array)

    def resident_blocks(self, name, block, waves_per_cu=None):
        """Size of a persistent grid: every workgroup must be resident.
        ``waves_per_cu`` caps it below what occupancy allows."""
        blocks = self.device.resident_blocks(self.module.kernel(name), block)
        waves_per_block = max(1, (block + 63) // 64)
        if waves_per_block % 4 and waves_per_block > 4:
            # the occupancy query counts wavefronts per CU; a workgroup whose
            # wavefronts do not divide over the four SIMDs takes the larger
            # share on some of them, and fewer such workgroups fit than the
            # total suggests (measured: 4 promised, 3 resident at 6 per group)
            per_cu = blocks // max(self.device.props.compute_units, 1)
            per_simd = per_cu * waves_per_block // 4
            fit = per_simd // -(-waves_per_block // 4)
            blocks = max(1, min(per_cu, fit)) * self.device.props.compute_units
        if waves_per_cu:
            # (a fraction leaves CUs without a workgroup: narrow DAGs)
            cap = -(-int(self.device.props.compute_units
                         * float(waves_per_cu)) // waves_per_block)
            blocks = min(blocks, max(cap, 1))
        return blocks

    def launch(self, name, grid, block, args):
        kernel = self.module.kernel(name)
        timing = getattr(self.device, "kernel_timing", None)
        if timing is None or timing.get("name") != name:
            self.device.launch(kernel, grid, block, args)
            return
        # measurement hook (eager launches only): events around this kernel
        start, stop = self.device.event(), self.device.event()
        self.device.record(start)
        self.device.launch(kernel, grid, block, args)
        self.device.record(stop)
        timing.setdefault("events", []).append((start, stop))

    def launch_levels(self, name, host_ptr, tasks_per_block, block, args,
                      start_index, end_index):
        self.device.launch_levels(
            self.module.kernel(name), host_ptr, tasks_per_block, block, args,
            start_index, end_index)


@dataclass
class HIPPreparedArguments:
    """Host/device values ordered for a generated HIP launcher."""

    launcher_argument_names: tuple
    values: dict
    host_values: dict
    lifted_variables: tuple
    device: object = None
    module: object = None
    zero_on_launch: tuple = ()
    graph: object = None
    workspace: dict = None
    graph_key: tuple = None

    @property
    def launcher_arguments(self):
        return tuple(self.values[name] for name in self.launcher_argument_names)

    def copy_to_host(self, name):
        if name not in self.values:
            raise HIPRuntimePreparationError(
                f"Unknown prepared HIP argument {name!r}.")
        value = self.values[name]
        copy_method = getattr(value, "copy_to_host", None)
        return copy_method() if copy_method is not None else value

    def copy_lifted_variables_to_host(self):
        return {name: self.copy_to_host(name) for name in self.lifted_variables}


def evaluate_host_prelude(lowering, argument_values, function_globals=None,
                          skip=()):
    """Evaluate removed host statements and return their named values
    (compiler/cuda_runtime.py:184-264).  Names in ``skip`` are not executed
    (device-side zero initialisation replaces them)."""
    statements = [
        s for s in lowering.host_prelude
        if not (isinstance(s, ast.Assign) and len(s.targets) == 1
                and isinstance(s.targets[0], ast.Name)
                and s.targets[0].id in skip)]
    if not statements:
        return {}
    namespace = dict(function_globals or {})
    namespace.update(argument_values)
    module = ast.fix_missing_locations(
        ast.Module(body=deepcopy(statements), type_ignores=[]))
    exec(compile(module, "<hip-host-prelude>", "exec"), namespace, namespace)
    stored = []
    for statement in statements:
        for node in ast.walk(statement):
            if (isinstance(node, ast.Name) and isinstance(node.ctx, ast.Store)
                    and node.id not in stored):
                stored.append(node.id)
    missing = [name for name in lowering.lifted_variables
               if name not in namespace and name not in skip]
    if missing:
        raise HIPRuntimePreparationError(
            "The removed host prelude did not define lifted variables: "
            + ", ".join(missing))
    return {name: namespace[name] for name in stored if name in namespace}


def _execution_values(execution_mode, execution_data):
    """Executor arrays by argument name (compiler/cuda_runtime.py:336-375)."""
    mode = execution_mode.replace("-", "_")
    if isinstance(execution_data, WarpTaskExecutionData):
        values = {
            "task_nodes": execution_data.task_nodes,
            "task_ptr": execution_data.task_ptr,
            "band_ptr": execution_data.band_ptr,
            "dep_count": execution_data.dep_count,
            "initial_dep_count": (
                execution_data.initial_dep_count
                if execution_data.initial_dep_count is not None
                else execution_data.dep_count),
            "dag_ptr": execution_data.dag_ptr,
            "dag_index": execution_data.dag_index,
        }
    elif mode == "sync_free":
        # The persistent executor needs its tasks in topological (level)
        # order for forward progress; plain successor/counter data has none.
        raise HIPRuntimePreparationError(
            "Sync-free HIP executors need level-ordered task data "
            "(WarpTaskExecutionData from preprocess_warp_tasks or the device "
            "inspector); got " + type(execution_data).__name__ + ".")
    elif mode == "wavefront":
        if not isinstance(execution_data, WavefrontExecutionData):
            raise HIPRuntimePreparationError(
                "Wavefront lowering requires WavefrontExecutionData.")
        values = {"wavefronts": execution_data.wavefronts,
                  "wavefront_ptr": execution_data.wavefront_ptr,
                  "task_nodes": execution_data.wavefronts,
                  "task_ptr": None,
                  "band_ptr": execution_data.wavefront_ptr}
    else:
        values = {}
    auxiliary = getattr(execution_data, "auxiliary_values", {}) or {}
    collisions = set(values) & set(auxiliary)
    if collisions:
        raise HIPRuntimePreparationError(
            "Auxiliary values conflict with executor arguments: "
            + ", ".join(sorted(collisions)))
    values.update(auxiliary)
    return values


WATCHDOG_UNIT_TICKS = 1 << 20        # of the 100 MHz device wall clock


def watchdog_budget(lowering, execution_data):
    """Time budget of one launch of a persistent executor for this plan, in
    units of 2^20 ticks of the 100 MHz wall clock (about 10.5 ms): two
    seconds plus 8 us per level of the DAG (per node for chain tasks, which
    run their members one after the other) plus 0.1 us per task (a wide DAG
    of few levels takes its time too), at most five minutes.  A stuck
    schedule on a DAG of a few hundred levels then gives up after two seconds
    instead of the twenty-odd the poll count alone took, and a chain of
    millions of levels, whose launch legitimately runs for seconds, keeps
    the time it needs.  ``watchdog_seconds`` of the lowering replaces the
    figure (a GPU shared with other work wants more); 0 there, a
    ``spin_limit`` the caller chose, or an unknown depth give 0: no time
    budget, the poll count alone ends a wait that cannot end."""
    from lcd_amd.hip_emitter import DEFAULT_SPIN_LIMIT
    chosen = getattr(lowering, "watchdog_seconds", None)
    if chosen is not None:
        if chosen <= 0:
            return 0
        return int(min(float(chosen), 3600.0) * 1.0e8 / WATCHDOG_UNIT_TICKS) + 1
    if getattr(lowering, "spin_limit", DEFAULT_SPIN_LIMIT) != DEFAULT_SPIN_LIMIT:
        return 0
    bands = getattr(execution_data, "band_ptr", None)
    if bands is None:
        bands = getattr(execution_data, "wavefront_ptr", None)
    try:
        depth = len(bands) - 1
        nodes = getattr(execution_data, "task_nodes", None)
        chains = getattr(execution_data, "task_ptr", None)
        tasks = len(nodes) if nodes is not None else 0
        if (nodes is not None and chains is not None
                and len(chains) - 1 != len(nodes)):
            depth = len(nodes)
    except TypeError:
        return 0
    seconds = min(2.0 + 8.0e-6 * max(depth, 0) + 1.0e-7 * max(tasks, 0), 300.0)
    return int(seconds * 1.0e8 / WATCHDOG_UNIT_TICKS) + 1


def _scalar_ctype(value):
    if isinstance(value, (bool, np.bool_)):
        return "long long"
    if isinstance(value, (int, np.integer)):
        return "long long"
    if isinstance(value, (float, np.floating)):
        return "double"
    return None


def prepare_hip_arguments(lowering, argument_values, execution_data,
                          function_globals=None, hip_module=None,
                          compiled_module=None, workspace=None):
    """Create lifted locals and device copies of every launcher argument.

    Mirrors ``prepare_cuda_arguments`` (compiler/cuda_runtime.py:128-181).
    ``hip_module`` is the device layer (default: the process GPU context).
    Differences: arrays already on the device pass through uncopied, lifted
    ``np.zeros`` arrays are created on the device, the mutable executor state
    (``dep_count``, ``task_counter``, ``done``, status word) lives in
    per-plan device buffers, and ``workspace`` (a dict) lets repeated calls
    reuse device buffers so a captured graph stays valid.
    """
    device = hip_module if hip_module is not None else default_device()
    workspace = workspace if workspace is not None else {}
    host_values = dict(argument_values)
    zero_names = tuple(lowering.zero_initialised)
    host_values.update(evaluate_host_prelude(
        lowering, host_values, function_globals, skip=zero_names))
    zero_arrays = {}
    for name, shape_source in lowering.zero_initialised.items():
        namespace = dict(function_globals or {})
        namespace.update(host_values)
        shape = eval(shape_source, namespace)
        shape = (int(shape),) if np.isscalar(shape) else tuple(shape)
        cached = workspace.get(("zero", name))
        if cached is None or cached.shape != shape:
            cached = device.empty(shape, np.float64)
            workspace[("zero", name)] = cached
        zero_arrays[name] = cached
        host_values[name] = cached
    execution_values = _execution_values(lowering.execution_mode, execution_data)
    host_values.update(execution_values)

    # structure arrays in task order (once per plan: the workspace keeps them)
    for name, source, offset in getattr(lowering, "queue_node_loads", ()):
        cached = workspace.get(("queue", name))
        if cached is None:
            cached = device.gather_int32(host_values[source],
                                         host_values["task_nodes"], offset)
            workspace[("queue", name)] = cached
        host_values[name] = cached

    # mutable executor state
    n_tasks = None
    for key in ("dep_count", "task_nodes", "wavefronts"):
        if key in execution_values:
            n_tasks = len(execution_values[key])
            break
    if lowering.execution_mode == "sync_free":
        initial = host_values.get("initial_dep_count")
        if "dep_count" in lowering.launcher_arguments:
            cached = workspace.get(("state", "dep_count"))
            if cached is None or len(cached) != len(initial):
                cached = device.empty((len(initial),), np.int32)
                workspace[("state", "dep_count")] = cached
            host_values["dep_count"] = cached
        if "done" in lowering.launcher_arguments:
            cached = workspace.get(("state", "done"))
            if cached is None or len(cached) != n_tasks:
                cached = device.empty((n_tasks,), np.int32)
                workspace[("state", "done")] = cached
            host_values["done"] = cached
        if "_lcd_mailbox" in lowering.launcher_arguments:
            # one slot per message: out_slot holds the slots 0 .. count-1
            slots = max(len(host_values["_lcd_in_pos"]), 1)
            cached = workspace.get(("state", "_lcd_mailbox"))
            if cached is None or len(cached) != slots:
                cached = device.empty((slots,), np.float64)
                workspace[("state", "_lcd_mailbox")] = cached
            host_values["_lcd_mailbox"] = cached
        if "_lcd_pub" in lowering.launcher_arguments:
            # final values of the published array, one slot per element
            slots = max(len(host_values[lowering.published_array]), 1)
            cached = workspace.get(("state", "_lcd_pub"))
            if cached is None or len(cached) != slots:
                cached = device.empty((slots,), np.float64)
                workspace[("state", "_lcd_pub")] = cached
            host_values["_lcd_pub"] = cached
        if "_lcd_xq" in lowering.launcher_arguments:
            # the value-as-flag copy in queue order, one slot per task
            cached = workspace.get(("state", "_lcd_xq"))
            if cached is None or len(cached) != max(n_tasks, 1):
                cached = device.empty((max(n_tasks, 1),), np.float64)
                workspace[("state", "_lcd_xq")] = cached
            host_values["_lcd_xq"] = cached
        for name in lowering.launcher_arguments:
            if not name.startswith("_lcd_staged_"):
                continue
            # position-indexed operands gathered into consumer order
            dtype = (np.int32 if lowering.array_arguments.get(name) == "int"
                     else np.float64)
            slots = max(len(host_values["_lcd_in_pos"]), 1)
            cached = workspace.get(("state", name))
            if cached is None or len(cached) != slots or (
                    cached.dtype != dtype):
                cached = device.empty((slots,), dtype)
                workspace[("state", name)] = cached
            host_values[name] = cached
        if getattr(lowering, "grid_sweep", None):
            host_values.update(_sweep_buffers(lowering, device, workspace))
        for name in ("task_counter", STATUS_ARGUMENT):
            cached = workspace.get(("state", name))
            if cached is None:
                if name == STATUS_ARGUMENT and hasattr(device, "to_device"):
                    # word 0: abort flag; word 1: time budget of this plan
                    cached = device.to_device(np.array(
                        [0, watchdog_budget(lowering, execution_data),
                         0, 0], dtype=np.int32))
                else:
                    cached = device.zeros((4,), np.int32)
                workspace[("state", name)] = cached
            host_values[name] = cached

    if getattr(lowering, "level_records", False):
        # operands of the records' edges, node values and the copy of the
        # array the tasks write, all in level order
        lanes = int(lowering.task_record_lanes or 1)
        for name in lowering.launcher_arguments:
            if not (name.startswith(("_lcd_lr_", "_lcd_lv_"))
                    or name == "_lcd_xq"):
                continue
            dtype = (np.int32 if lowering.array_arguments.get(name) == "int"
                     else np.float64)
            slots = max(n_tasks, 1) * (lanes if name.startswith("_lcd_lr_")
                                       else 1)
            cached = workspace.get(("state", name))
            if cached is None or len(cached) != slots or (
                    cached.dtype != dtype):
                cached = device.empty((slots,), dtype)
                workspace[("state", name)] = cached
            host_values[name] = cached

    missing = [name for name in lowering.launcher_arguments
               if name not in host_values]
    if missing:
        raise HIPRuntimePreparationError(
            "Values are missing for generated launcher arguments: "
            + ", ".join(missing))

    prepared = {}
    for name in lowering.launcher_arguments:
        value = host_values[name]
        if name in HOST_LAUNCH_ARGUMENTS:
            if is_device_array(value):
                value = value.copy_to_host()
            prepared[name] = np.ascontiguousarray(value, dtype=np.int32)
        else:
            prepared[name] = _prepare_value(
                name, value, device, workspace, lowering)

    module = None
    if compiled_module is not None:
        module = _load_for_values(compiled_module, lowering, prepared, device)
    if (getattr(lowering, "restage_launcher_name", None) and module is not None
            and isinstance(device, HIPDevice)):
        # the matrix's share of the staged records (grid sweep, level
        # records): staged again when the contents of its arrays have
        # changed since the last time
        digests = tuple(device.digest(prepared[name])
                        for name in lowering.stage_static_arrays)
        if workspace.get(("sweep", "digests")) != digests:
            stage_static_values(compiled_module, lowering, prepared, module,
                               device)
            workspace[("sweep", "digests")] = digests
    # a captured graph stays valid while every pointer and scalar is unchanged
    graph_key = ("graph", lowering.kernel_name) + tuple(
        (name, device_pointer(value)) if is_device_array(value)
        else (name, value.tobytes()) if isinstance(value, np.ndarray)
        else (name, value)
        for name, value in prepared.items())
    return HIPPreparedArguments(
        launcher_argument_names=tuple(lowering.launcher_arguments),
        values=prepared, host_values=host_values,
        lifted_variables=tuple(lowering.lifted_variables), device=device,
        module=module,
        zero_on_launch=tuple(
            name for name in zero_arrays
            if name not in getattr(lowering, "executor_initialised", ())),
        graph=workspace.get(graph_key), workspace=workspace,
        graph_key=graph_key)


def _prepare_value(name, value, device, workspace, lowering):
    if is_device_array(value) or value is None:
        return value
    if isinstance(value, (bool, np.bool_)):
        return int(value)
    if np.isscalar(value):
        return value.item() if isinstance(value, np.generic) else value
    if isinstance(value, (list, tuple)):
        value = np.asarray(value)
    if isinstance(value, np.ndarray):
        if value.dtype == np.int64 and lowering.array_arguments.get(name) == "int" \
                and name in ("task_nodes", "task_ptr", "dag_ptr", "dag_index",
                             "initial_dep_count"):
            value = value.astype(np.int32)
        cached = workspace.get(("upload", name))
        result = device.to_device(value, into=cached)
        workspace[("upload", name)] = result
        return result
    raise HIPRuntimePreparationError(
        "HIP launcher arguments must be scalars, NumPy arrays, sequences, "
        f"or existing device arrays; received {type(value).__name__}.")


def _kernel_signature_types(lowering, prepared):
    """Concrete C types of every kernel argument for these values."""
    array_types, scalar_types = _default_types(lowering)
    for name in lowering.kernel_arguments:
        value = prepared.get(name)
        if name in lowering.array_arguments:
            if value is not None and is_device_array(value):
                _, dtype = device_array_meta(value)
                ctype = _DTYPE_TO_C.get(dtype.name)
                if ctype is None:
                    raise HIPRuntimePreparationError(
                        f"Unsupported dtype {dtype} for array {name!r}.")
                array_types[name] = ctype
        elif name in lowering.scalar_arguments and name in prepared:
            if value is not None and is_device_array(value):
                scalar_types[name] = "const void*"
            elif value is None:
                scalar_types[name] = "const void*"
            else:
                ctype = _scalar_ctype(value)
                if ctype is None:
                    raise HIPRuntimePreparationError(
                        f"Unsupported scalar {name!r}: {type(value).__name__}.")
                if name not in ("band_start", "band_end", "task_count"):
                    scalar_types[name] = ctype
    return array_types, scalar_types


def _load_for_values(compiled, lowering, prepared, device):
    array_types, scalar_types = _kernel_signature_types(lowering, prepared)
    default_arrays, default_scalars = _default_types(lowering)
    options = []
    for name in lowering.kernel_arguments:
        if name in array_types and array_types[name] != default_arrays.get(name):
            options.append(f"-DLCD_T_{name}={array_types[name]}")
        if name in scalar_types and scalar_types[name] != default_scalars.get(name):
            options.append(f"-DLCD_T_{name}={scalar_types[name]}")
    key = tuple(options)
    cache_key = (id(device), key)
    if cache_key not in compiled.loaded:
        code = compiled.code_for(key)
        ctypes_of = []
        for name in lowering.kernel_arguments:
            if name in array_types:
                ctypes_of.append(ctypes.c_void_p)
            else:
                text = scalar_types[name]
                ctypes_of.append(ctypes.c_void_p if text == "const void*"
                                 else _CTYPES[text])
        argument_ctypes = {lowering.kernel_name: ctypes_of}
        if lowering.reset_kernel_name:
            if lowering.dependence_protocol in ("pull", "mailbox"):
                reset = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]
            else:
                reset = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                         ctypes.c_int64]
            argument_ctypes[lowering.reset_kernel_name] = reset
        if getattr(lowering, "stage_kernel_name", None):
            stage = []
            for name in lowering.stage_kernel_arguments:
                if name in scalar_types:
                    text = scalar_types[name]
                    stage.append(ctypes.c_void_p if text == "const void*"
                                 else _CTYPES[text])
                else:
                    stage.append(ctypes.c_void_p)
            argument_ctypes[lowering.stage_kernel_name] = stage + [
                ctypes.c_int64]
        for name in getattr(lowering, "stage_kernels", ()):
            # the staging kernels of the grid sweep share the signature
            argument_ctypes[name] = list(ctypes_of)
        compiled.loaded[cache_key] = device.load_module(code, argument_ctypes)
    return compiled.loaded[cache_key]


EMPTY_MARKER_WORD = 0x7FF84C43       # both halves of the empty marker (a NaN)


def _sweep_buffers(lowering, device, workspace):
    """Device memory of the grid sweep, once per plan: the records in the
    wavefronts' order, the solution in the same order, the faces between
    workgroups (every slot the empty marker: a slot is filled and emptied
    again within one launch) and the two counters of a launch."""
    geometry = lowering.grid_sweep
    cached = workspace.get(("sweep", "buffers"))
    if cached is None:
        slots = geometry["slots"]
        faces = geometry["bundles"] + geometry["nby"] + 1
        cached = {
            "_lcd_sw_ops": device.empty((slots // 64 * geometry["record"],),
                                        np.float64),
            "_lcd_sw_out": device.empty((slots,), np.float64),
            "_lcd_sw_yface": device.empty(
                (faces * geometry["yrows"] * geometry["wz"],), np.float64),
            "_lcd_sw_zface": device.empty(
                (faces * geometry["zrows"] * geometry["wy"],), np.float64),
            "_lcd_sw_claim": device.zeros((4,), np.int32),
        }
        workspace[("sweep", "buffers")] = cached
        _sweep_reset(cached, device)
    return cached


def _sweep_reset(buffers, device):
    """Every face slot empty, both counters zero: the state a launch of
    the sweep starts from and, unless it is abandoned, ends in."""
    if not isinstance(device, HIPDevice):
        return
    for name in ("_lcd_sw_yface", "_lcd_sw_zface"):
        array = buffers[name]
        _check(device.lib.lcdhip_buffer_fill32(
            ctypes.c_void_p(array.pointer), ctypes.c_uint32(EMPTY_MARKER_WORD),
            ctypes.c_size_t(array.nbytes // 4), device.stream))
    device.fill_zero(buffers["_lcd_sw_claim"])


def stage_static_values(compiled_module, lowering, prepared_values, module,
                       device):
    """Lay the matrix's share of the grid sweep's records out again (the
    coefficients by direction, the node loads that come from the matrix
    arrays, the prepared reciprocals): to be called whenever the contents of
    ``lowering.stage_static_arrays`` have changed."""
    launcher = compiled_module.namespace[lowering.restage_launcher_name]
    context = LaunchContext(device, module, None)
    launcher(context, *[prepared_values[name]
                        for name in lowering.launcher_arguments])


# A captured level loop is one graph with a kernel node per level.  Replaying
# such a graph of about three thousand nodes under rocprofv3's kernel trace
# ended in a segmentation fault inside hipGraphLaunch once (the same graph
# replays correctly without the tracer, graphs of a few hundred nodes replay
# correctly with it, and nothing of this library is dereferenced during the
# launch), and no cause could be shown.  With a rocprofiler tool library
# loaded, level loops beyond this many launches are therefore issued eagerly.
TRACED_GRAPH_NODE_LIMIT = 1024
_traced_graph_notice = []


def profiler_attached():
    """True when the process was started under rocprofv3 (its tool library
    is named in the environment it sets up)."""
    return bool(os.environ.get("ROCP_TOOL_LIBRARIES")) or (
        "rocprofiler" in os.environ.get("LD_PRELOAD", ""))


def _level_launches(lowering, prepared):
    if getattr(lowering, "execution_mode", None) != "wavefront":
        return 0
    for name in ("band_ptr", "wavefront_ptr"):
        pointers = prepared.values.get(name)
        if pointers is None:
            pointers = prepared.host_values.get(name)
        if pointers is not None and hasattr(pointers, "__len__"):
            return max(len(pointers) - 1, 0)
    return 0


def launch_hip_call(compiled_module, lowering, prepared_arguments,
                    use_graph=True):
    """Enqueue one execution of the prepared call (no host synchronisation).

    Lifted zero-initialised arrays are cleared on the device first.  The
    whole sequence (clears, resets, level launches) is captured into a
    hipGraph on the first call and replayed afterwards.
    """
    prepared = prepared_arguments
    device = prepared.device
    module = prepared.module
    if module is None and hasattr(device, "load_module"):
        module = _load_for_values(compiled_module, lowering, prepared.values,
                                  device)
        prepared.module = module
    real_device = isinstance(device, HIPDevice)
    if (use_graph and real_device and profiler_attached()
            and _level_launches(lowering, prepared)
            > TRACED_GRAPH_NODE_LIMIT):
        if not _traced_graph_notice:
            _traced_graph_notice.append(True)
            print(f"lcd_amd: a profiler is attached; the level loop of "
                  f"{lowering.function_name} "
                  f"({_level_launches(lowering, prepared)} launches) is "
                  "issued eagerly instead of replayed from a graph",
                  file=sys.stderr, flush=True)
        use_graph = False
    if use_graph and real_device and prepared.graph is not None:
        prepared.graph.launch(device.stream)
        return

    def enqueue():
        for name in prepared.zero_on_launch:
            device.fill_zero(prepared.values[name])
        context = LaunchContext(device, module, None)
        compiled_module.launcher(context, *prepared.launcher_arguments)

    if use_graph and real_device:
        device.begin_capture()
        try:
            enqueue()
        finally:
            graph = device.end_capture()
        prepared.graph = graph
        if prepared.workspace is not None:
            for key in [k for k in prepared.workspace
                        if isinstance(k, tuple) and k and k[0] == "graph"]:
                prepared.workspace.pop(key).destroy()
            prepared.workspace[prepared.graph_key] = graph
        graph.launch(device.stream)
    else:
        enqueue()


def check_executor_status(lowering, prepared_arguments):
    """Raise if a sync-free executor tripped its watchdog, and re-arm it."""
    status = prepared_arguments.values.get(STATUS_ARGUMENT)
    if status is None:
        return
    host = status.copy_to_host()
    if int(host[0]) != 0:
        # re-arm the flag; the plan's time budget in word 1 stays
        device = prepared_arguments.device
        _check(device.lib.lcdhip_buffer_fill32(
            ctypes.c_void_p(status.pointer), ctypes.c_uint32(0),
            ctypes.c_size_t(1), device.stream))
        if getattr(lowering, "grid_sweep", None):
            # an abandoned launch leaves faces and counters half used
            _sweep_reset({name: prepared_arguments.values[name]
                          for name in ("_lcd_sw_yface", "_lcd_sw_zface",
                                       "_lcd_sw_claim")}, device)
            if int(host[0]) == 3:
                raise HIPRuntimeError(
                    f"The grid sweep of {lowering.function_name} met an "
                    "incoming entry that is not one step down along an axis "
                    "of the grid.  The result is not valid; run with "
                    "grid_sweep=False.", ERR_ARGUMENT)
        if int(host[0]) == 2 and getattr(lowering, "band_walker", False):
            raise HIPRuntimeError(
                f"The band walker of {lowering.function_name} met an edge its "
                "table has no cell for: one that spans 64 iterations or "
                "more, or a second edge between the same two iterations. "
                "The result is not valid; run with band_walker=False.",
                ERR_ARGUMENT)
        raise ExecutorWatchdogError(
            f"The sync-free executor of {lowering.function_name} gave up "
            "waiting for a dependence (cyclic or inconsistent schedule).",
            ERR_WATCHDOG)


def execute_hip_call(compiled_module, lowering, prepared_arguments,
                     function_globals=None, use_graph=True):
    """Launch prepared work and restore the original return semantics
    (compiler/cuda_runtime.py:202-228)."""
    launch_hip_call(compiled_module, lowering, prepared_arguments, use_graph)
    device = prepared_arguments.device
    if device is None or not hasattr(device, "synchronize"):
        raise HIPRuntimePreparationError(
            "The device layer does not provide synchronize().")
    device.synchronize()
    check_executor_status(lowering, prepared_arguments)
    result_values = dict(prepared_arguments.host_values)
    for name in _returned_names(lowering.host_epilogue):
        if name in prepared_arguments.values:
            result_values[name] = prepared_arguments.copy_to_host(name)
    # lifted arrays the epilogue may use; a returned one is already there
    for name in prepared_arguments.lifted_variables:
        if name not in result_values or (
                name in prepared_arguments.values
                and result_values[name] is prepared_arguments.values[name]):
            result_values[name] = prepared_arguments.copy_to_host(name)
    return _evaluate_host_epilogue(lowering, result_values,
                                   function_globals or {})


def _returned_names(statements):
    names = []
    for statement in statements:
        for node in ast.walk(statement):
            if not isinstance(node, ast.Return) or node.value is None:
                continue
            for value_node in ast.walk(node.value):
                if (isinstance(value_node, ast.Name)
                        and isinstance(value_node.ctx, ast.Load)
                        and value_node.id not in names):
                    names.append(value_node.id)
    return names


def _evaluate_host_epilogue(lowering, result_values, function_globals):
    if not lowering.host_epilogue:
        return None
    namespace = dict(function_globals)
    namespace.update(result_values)
    helper = "_generated_hip_host_epilogue"
    function = ast.FunctionDef(
        name=helper,
        args=ast.arguments(posonlyargs=[], args=[], kwonlyargs=[],
                           kw_defaults=[], defaults=[]),
        body=deepcopy(lowering.host_epilogue), decorator_list=[], returns=None,
        type_comment=None)
    module = ast.fix_missing_locations(
        ast.Module(body=[function], type_ignores=[]))
    exec(compile(module, "<hip-host-epilogue>", "exec"), namespace, namespace)
    return namespace[helper]()

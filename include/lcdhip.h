/*
 * lcdhip.h -- C ABI of liblcdhip.so, the MI355X (gfx950) execution backend
 * behind LCD's `@parallel` decorator.
 *
 * Everything the reference does between "the decorated function is called
 * with host CSR/CSC arrays" and "the result array is back on the host" goes
 * through these entry points: device buffers and copies, run-time compilation
 * and launch of the generated HIP kernels, the level loop of the wavefront
 * executor, and the on-device DAG inspector (edges, in-degrees, level sets,
 * structural lookup tables).
 *
 * Conventions
 *   - every function returns 0 (LCDHIP_OK) or a positive LCDHIP_ERR_* code;
 *     lcdhip_last_error() returns a thread-local message for the last failure
 *   - the library never frees or keeps caller memory; every *_create/_alloc/
 *     _build/_compile/_load has a matching *_destroy/_free
 *   - pointers named d_* are device pointers; stream arguments are opaque
 *     handles from lcdhip_stream_create (NULL = the library's default stream)
 *   - not re-entrant: one host thread drives one context
 *
 * The citations name the reference code (paths under the reference checkout)
 * that each entry point replaces.
 */
#ifndef LCDHIP_H
#define LCDHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LCDHIP_OK 0
#define LCDHIP_ERR_HIP 1          /* a HIP runtime call failed */
#define LCDHIP_ERR_COMPILE 2      /* hiprtc rejected the generated source */
#define LCDHIP_ERR_ARGUMENT 3     /* bad argument / handle */
#define LCDHIP_ERR_DAG_BOUNDS 4   /* DAG endpoint outside [0, n) */
#define LCDHIP_ERR_DAG_CYCLE 5    /* level sets do not cover every node */
#define LCDHIP_ERR_LOOKUP_POINTER 6 /* non-monotone / out-of-range pointers */
#define LCDHIP_ERR_LOOKUP_ORDER 7   /* unsorted segment */
#define LCDHIP_ERR_WATCHDOG 8     /* a spin-wait executor gave up */
#define LCDHIP_ERR_NO_DEVICE 9    /* no usable GPU */

typedef struct lcdhip_module lcdhip_module;
typedef struct lcdhip_kernel lcdhip_kernel;
typedef struct lcdhip_graph lcdhip_graph;
typedef struct lcdhip_dag lcdhip_dag;
typedef void *lcdhip_stream;
typedef void *lcdhip_event;

const char *lcdhip_last_error(void);
const char *lcdhip_version(void);

/* ------------------------------------------------------------- context ---
 * Replaces the implicit numba.cuda context (compiler/cuda_runtime.py:141-142,
 * compiler/scheduler.py:714-736). */
int lcdhip_init(int device);
int lcdhip_shutdown(void);
int lcdhip_device_count(int *count);

typedef struct {
    int32_t compute_units;        /* 256 on MI355X */
    int32_t xcd_count;            /* 8 */
    int32_t wavefront_size;       /* 64 */
    int32_t max_threads_per_block;
    int32_t lds_bytes_per_block;
    int32_t lds_bytes_per_cu;
    int32_t clock_khz;
    int32_t memory_clock_khz;
    int32_t memory_bus_bits;
    int32_t l2_bytes;
    int64_t global_memory_bytes;
    char name[128];
    char arch[64];
} lcdhip_props;
int lcdhip_device_props(lcdhip_props *out);

/* Measured machine constants for the analytic scheduler; replaces
 * measure_arch_constants / _measure_launch_latency / _measure_atomic_cost
 * (compiler/scheduler.py:714-775).  handoff_s is the latency of one
 * release->acquire hop between two workgroups through device-scope atomics,
 * barrier_s one grid-wide barrier of a resident persistent grid. */
typedef struct {
    double launch_latency_s;
    double atomic_cost_s;
    double memory_bandwidth_bytes_per_s;
    double lane_flops_per_s;
    double handoff_s;
    double barrier_s;
    double graph_node_s;
    /* the same hop between two wavefronts of ONE workgroup through LDS, and
     * one step of a chain of dependent fp64 tasks x = (b - c * x) / d in one
     * lane: what a dependence costs when its hand-off is free, the floor of
     * levels x step under every executor (no counterpart in the reference) */
    double lds_handoff_s;
    double chain_step_s;
} lcdhip_arch;
int lcdhip_measure_arch(lcdhip_arch *out);

/* ------------------------------------------------- buffers and streams ---
 * Replace cuda.to_device / copy_to_host / cuda.synchronize
 * (compiler/cuda_runtime.py:391-401, 47-55, 215). */
int lcdhip_buffer_alloc(size_t bytes, void **d_out);
int lcdhip_buffer_free(void *d_ptr);
int lcdhip_buffer_upload(void *d_dst, const void *host_src, size_t bytes,
                         lcdhip_stream stream);
int lcdhip_buffer_download(void *host_dst, const void *d_src, size_t bytes,
                           lcdhip_stream stream);
int lcdhip_buffer_copy(void *d_dst, const void *d_src, size_t bytes,
                       lcdhip_stream stream);
/* Fill with a 32-bit pattern using a kernel (safe inside graph capture). */
int lcdhip_buffer_fill32(void *d_dst, uint32_t value, size_t count,
                         lcdhip_stream stream);
int lcdhip_host_alloc(size_t bytes, void **host_out);   /* pinned */
int lcdhip_host_free(void *host_ptr);
int lcdhip_stream_create(lcdhip_stream *out);
int lcdhip_stream_destroy(lcdhip_stream stream);
int lcdhip_stream_sync(lcdhip_stream stream);
int lcdhip_event_create(lcdhip_event *out);
int lcdhip_event_destroy(lcdhip_event event);
int lcdhip_event_record(lcdhip_event event, lcdhip_stream stream);
int lcdhip_event_elapsed_ms(lcdhip_event start, lcdhip_event stop, float *ms);

/* -------------------------------------------------- generated modules ---
 * Replace compile_cuda_module and the numba JIT behind it
 * (compiler/cuda_runtime.py:70-125).  lcdhip_module_compile_code needs no
 * GPU (hiprtc cross-compiles for gfx950); lcdhip_module_load needs one. */
int lcdhip_module_compile_code(const char *source, const char *name,
                               const char *const *options, int option_count,
                               void **code_out, size_t *size_out,
                               char **log_out);
void lcdhip_free_host(void *ptr); /* frees code_out / log_out */
int lcdhip_module_load(const void *code, size_t size, lcdhip_module **out);
int lcdhip_module_destroy(lcdhip_module *module);
int lcdhip_module_get_kernel(lcdhip_module *module, const char *name,
                             lcdhip_kernel **out);
/* Largest co-resident grid of `kernel` at this block size (for persistent
 * executors: every workgroup must be able to make progress). */
int lcdhip_kernel_max_resident_blocks(lcdhip_kernel *kernel, int block_threads,
                                      size_t lds_bytes, int *blocks_out);

/* One launch; replaces kernel[grid, block](*args) in the generated launchers
 * (compiler/cuda_lowering.py:673-735).  args[k] points at the value of the
 * k-th kernel parameter. */
int lcdhip_launch(lcdhip_kernel *kernel, uint32_t grid_x, uint32_t block_x,
                  size_t lds_bytes, lcdhip_stream stream, void **args);

/* The host level loop of the wavefront launchers
 * (compiler/cuda_lowering.py:855-1068): for every level/band l with
 * host_ptr[l] < host_ptr[l+1], set *(int32*)args[start_arg] = host_ptr[l],
 * *(int32*)args[end_arg] = host_ptr[l+1] and launch
 * ceil((host_ptr[l+1]-host_ptr[l]) / tasks_per_block) blocks.  There is no
 * host synchronisation between levels: stream order carries the dependence.
 * Intended to be issued once under graph capture and then replayed. */
int lcdhip_launch_levels(lcdhip_kernel *kernel, const int32_t *host_ptr,
                         int64_t level_count, int32_t tasks_per_block,
                         uint32_t block_x, size_t lds_bytes,
                         lcdhip_stream stream, void **args, int start_arg,
                         int end_arg);

/* hipGraph capture of a launcher body. */
int lcdhip_graph_begin_capture(lcdhip_stream stream);
int lcdhip_graph_end_capture(lcdhip_stream stream, lcdhip_graph **out);
int lcdhip_graph_launch(lcdhip_graph *graph, lcdhip_stream stream);
int lcdhip_graph_destroy(lcdhip_graph *graph);

/* ------------------------------------------------- on-device inspector ---
 * Replaces the generated Python `extract_dag` (compiler/dag_codegen.py:
 * 1151-1550, 1600-1618) and compiler/dag_preprocessing.py:94-255.
 *
 * One rule enumerates, for every task `seg` in [0, n):
 *     for p in [d_ptr[seg] + lower_offset, d_ptr[seg+1] + upper_offset):
 *         if break_at_owner and d_idx[p] >= seg: break
 *         (src, dst) = owner_is_source ? (seg, d_idx[p]) : (d_idx[p], seg)
 *         if guard(src, dst): edge src -> dst
 * guard: 0 none, 1 dst > src, 2 src != dst.
 *
 * A rule with relation LCDHIP_RULE_LATER has no structure arrays (d_ptr and
 * d_idx NULL, idx_size ignored) and enumerates
 *     for j in [seg + lower_offset, n): edge seg -> j      (lower_offset >= 1)
 * which is what the reference's planner emits for a relational loop such as
 * `for j in range(k + 1, n)` (CSC ILU0, compiler/demo/spilu0.py:50-82;
 * compiler/transform_tests/test_spilu0_codegen.py:146-150).  It yields
 * (n - lower_offset)(n - lower_offset + 1) / 2 edges, so it is meant for
 * small n; LCDHIP_DAG_INCOMING cannot be combined with it.
 *
 * A rule with relation LCDHIP_RULE_NEXT (no structure arrays either) yields
 * the single edge seg -> seg + lower_offset (lower_offset >= 1).  With
 * lower_offset == 1 it is the transitive reduction of the complete order:
 * what the inspector is given when a dependence could not be refuted and
 * cannot be enumerated either, the counterpart of the reference keeping every
 * dependence its solver does not refute in time
 * (compiler/legality_check.py:431-443).  Any n; no LCDHIP_DAG_INCOMING.
 */
#define LCDHIP_RULE_SEGMENT 0
#define LCDHIP_RULE_LATER 1
#define LCDHIP_RULE_NEXT 2
#define LCDHIP_GUARD_NONE 0
#define LCDHIP_GUARD_GREATER 1
#define LCDHIP_GUARD_NOT_EQUAL 2

typedef struct {
    const int32_t *d_ptr;
    const int32_t *d_idx;
    int64_t idx_size;
    int32_t owner_is_source;
    int32_t lower_offset;
    int32_t upper_offset;
    int32_t guard;
    int32_t break_at_owner;
    int32_t relation;        /* LCDHIP_RULE_SEGMENT, _LATER or _NEXT */
} lcdhip_dag_rule;

#define LCDHIP_DAG_LEVELS 1u        /* also build level sets / wavefronts */
#define LCDHIP_DAG_FORCE_KAHN 2u    /* use the frontier algorithm even when
                                       every edge goes low id -> high id */
#define LCDHIP_DAG_INCOMING 4u      /* also list, per destination, the
                                       positions p that produce its edges */

typedef struct {
    int64_t n;
    int64_t edges;           /* unique edges */
    int64_t levels;
    int64_t scheduled;       /* nodes covered by the level sets */
    int64_t max_level_width;
    int32_t topological_ids; /* 1 when every edge has src < dst */
    int32_t level_algorithm; /* 0 none, 1 frontier (Kahn), 2 ordered sweep */
} lcdhip_dag_info;

/* Arrays owned by the dag handle (all int32, device resident). */
#define LCDHIP_DAG_PTR 0            /* n + 1: CSR successor offsets */
#define LCDHIP_DAG_INDEX 1          /* edges: successors, sorted, unique */
#define LCDHIP_DAG_DEP_COUNT 2      /* n: unique in-degree */
#define LCDHIP_DAG_EDGE_COUNT 3     /* n: rule hits per destination */
#define LCDHIP_DAG_LEVEL_OF 4       /* n: level, -1 = unscheduled */
#define LCDHIP_DAG_WAVEFRONTS 5     /* scheduled: nodes by (level, id) */
#define LCDHIP_DAG_WAVEFRONT_PTR 6  /* levels + 1 */
/* With LCDHIP_DAG_INCOMING: for destination v the positions
 * in_pos[in_ptr[v] .. in_ptr[v+1]) of the rule's index array whose entries
 * produce an edge into v, ordered by (source, position), duplicates kept
 * (in_ptr is the scan of EDGE_COUNT).  Positions of rule r are offset by the
 * sum of idx_size of the rules before it.  out_slot is the inverse listing:
 * out_slot[in_pos[k]] = k, and -1 for positions that produce no edge; in_src[k]
 * is the source node of the edge in_pos[k] produces.  The
 * mailbox protocol delivers one message per position: the producer of
 * position p writes message slot out_slot[p], the consumer v reads slots
 * in_ptr[v] .. in_ptr[v+1) in order. */
#define LCDHIP_DAG_IN_PTR 7         /* n + 1 */
#define LCDHIP_DAG_IN_POS 8         /* candidate edges */
#define LCDHIP_DAG_OUT_SLOT 9       /* sum of idx_size over the rules */
#define LCDHIP_DAG_IN_SRC 10        /* candidate edges: source of in_pos[k] */
/* After lcdhip_dag_band_chains: */
#define LCDHIP_DAG_TASK_NODES 11    /* n: chain members, chain after chain */
#define LCDHIP_DAG_TASK_PTR 12      /* tasks + 1: chain offsets */
#define LCDHIP_DAG_BAND_PTR 13      /* bands + 1: first chain of every band */
/* After lcdhip_dag_tile_order: */
#define LCDHIP_DAG_TILE_NODES 14    /* n: nodes by (id / tile_rows, level, id) */
/* After lcdhip_dag_task_records (q = position in the task order): */
#define LCDHIP_DAG_REC_IN 15        /* 2 n: in_ptr[v], in_ptr[v + 1] of task q */
#define LCDHIP_DAG_REC_SRC 16       /* n * lanes: in_src of its first edges */
#define LCDHIP_DAG_REC_POS 17       /* n * lanes: in_pos of its first edges */
/* After lcdhip_dag_tile_order / lcdhip_dag_box_order: */
#define LCDHIP_DAG_TILE_POS 18      /* n: position of every node in TILE_NODES */
#define LCDHIP_DAG_ARRAYS 19

int lcdhip_dag_build(const lcdhip_dag_rule *rules, int rule_count, int64_t n,
                     uint32_t flags, lcdhip_stream stream, lcdhip_dag **out);
/* Chain tasks for band_width > 1 (replaces _band_chains,
 * compiler/dag_preprocessing.py:258-298): the level sets are cut into bands of
 * band_width consecutive levels; inside a band every connected component of
 * the DAG becomes one task whose members run in (level, id) order.  Chains are
 * listed band by band, inside a band by their first member.  Needs a dag built
 * with LCDHIP_DAG_LEVELS whose level sets cover every node.  May be called
 * again with another width; the previous chain arrays are released. */
int lcdhip_dag_band_chains(lcdhip_dag *dag, int64_t band_width,
                           lcdhip_stream stream, int64_t *tasks_out,
                           int64_t *bands_out);
/* Task order of the tiled persistent executor (no counterpart in the
 * reference: its executors have one global queue): nodes grouped into tiles of
 * tile_rows consecutive ids, inside a tile in (level, id) order.  With ids in
 * topological order (info.topological_ids) a tile depends on lower tiles only.
 * Needs LCDHIP_DAG_LEVELS and level sets that cover every node. */
int lcdhip_dag_tile_order(lcdhip_dag *dag, int64_t tile_rows,
                          lcdhip_stream stream);
/* Task order of the tiled persistent executor over boxes of a structured grid
 * (no counterpart in the reference): node id = x + grid[0] * (y + grid[1] * z);
 * the nodes of one box of box[0] x box[1] x box[2] grid points are listed
 * together, boxes in (z, y, x) order, inside a box in (level, id) order.  The
 * executor cuts the list into tiles of box[0] * box[1] * box[2] positions, so
 * with extents that divide the grid a tile is a box, and the hand-offs along
 * all three axes stay inside a workgroup except at box faces (consecutive ids
 * keep one axis at most).  Builds TILE_NODES and TILE_POS.  The list must be a
 * topological order for the executor to finish: lcdhip_dag_task_records with
 * LCDHIP_RECORDS_TILE_POSITIONS checks that and fails otherwise (any stencil
 * whose edges go from a lower to a higher id in natural order passes).
 * grid[0] * grid[1] * grid[2] must equal n. */
int lcdhip_dag_box_order(lcdhip_dag *dag, const int64_t grid[3],
                         const int64_t box[3], lcdhip_stream stream);
/* The distinct values of (destination - source) over the unique edges,
 * ascending, with the number of edges of each: what tells a structured grid
 * in natural order (a 7-point stencil has the offsets 1, nx, nx * ny) from a
 * general matrix.  Up to `capacity` values are written to the host arrays;
 * *distinct_out receives how many there are.  (Decision input of this
 * backend's scheduler; no counterpart in the reference.) */
int lcdhip_dag_edge_offsets(const lcdhip_dag *dag, int64_t capacity,
                            int64_t *offsets_out, int64_t *counts_out,
                            int64_t *distinct_out, lcdhip_stream stream);
/* Number of (unique) edges whose two endpoints lie in the same tile of
 * tile_rows consecutive ids: the share of hand-offs a tiled executor keeps
 * inside a workgroup.  (Decision input of this backend's scheduler; no
 * counterpart in the reference.) */
int lcdhip_dag_tile_locality(const lcdhip_dag *dag, int64_t tile_rows,
                             lcdhip_stream stream, int64_t *local_edges_out);
#define LCDHIP_RECORDS_LEVEL_ORDER 0     /* tasks in WAVEFRONTS order */
#define LCDHIP_RECORDS_TILE_ORDER 1      /* tasks in TILE_NODES order */
#define LCDHIP_RECORDS_TILE_POSITIONS 2  /* the same, sources as positions */
/* Fixed-size records of the incoming listing in the order the persistent
 * executor visits the tasks (`tiled` is one of LCDHIP_RECORDS_*; the tile
 * orders need lcdhip_dag_tile_order or lcdhip_dag_box_order first): for the
 * task at position q, REC_IN holds its range of the
 * incoming listing and REC_SRC / REC_POS[q * lanes + l] the source and the
 * position of its l-th incoming edge (0 beyond its in-degree).  With
 * LCDHIP_RECORDS_TILE_POSITIONS a source is named by its position in
 * TILE_NODES instead of its id (tiles that do not follow the ids address their
 * LDS copy that way), and the call fails when a source does not come before
 * its consumer in that order.  A wavefront
 * then fetches everything its tasks need to start polling with loads whose
 * addresses depend on q alone.  *overflow_tasks_out (may be NULL) receives
 * the number of tasks with more than `lanes` incoming edges, whose further
 * edges stay in the incoming listing only.  Needs LCDHIP_DAG_INCOMING and
 * LCDHIP_DAG_LEVELS; lanes in [1, 64].  (Layout of this backend's executor;
 * no counterpart in the reference.) */
int lcdhip_dag_task_records(lcdhip_dag *dag, int lanes, int tiled,
                            lcdhip_stream stream, int64_t *overflow_tasks_out);
int lcdhip_dag_get_info(const lcdhip_dag *dag, lcdhip_dag_info *out);
int lcdhip_dag_array(const lcdhip_dag *dag, int which, void **d_out,
                     int64_t *count_out);
int lcdhip_dag_download(const lcdhip_dag *dag, int which, int32_t *host_out,
                        int64_t capacity);
int lcdhip_dag_destroy(lcdhip_dag *dag);

/* Diagonal-position table; replaces _materialize_lookup
 * (compiler/structural_lookups.py:279-333).  d_positions[s] = first p in
 * [d_ptr[s], d_ptr[s+1]) with d_idx[p] == s, else -1. */
int lcdhip_lookup_build(const int32_t *d_ptr, const int32_t *d_idx, int64_t n,
                        int64_t idx_size, int32_t *d_positions,
                        lcdhip_stream stream);

/* Pair table of a segmented structure (d_ptr[n + 1], d_idx[idx_size], segments
 * sorted): for segment s with entries a, b in [0, len_s),
 * d_table[d_base[s] + a * len_s + b] = first position in segment
 * d_idx[d_ptr[s] + a] whose index equals d_idx[d_ptr[s] + b], or -1;
 * d_base[s] = sum of len^2 over the segments before s (n + 1 entries).  It
 * holds the results of the searches ILU0 makes per pivot and updated entry
 * (`for kj_ptr in range(A_indptr[k], A_indptr[k + 1]): if A_indices[kj_ptr] ==
 * j`, reference compiler/demo/spilu0.py:38-46): they depend on the structure
 * only, and read from a table their addresses depend on the task's own
 * positions alone.  Extends the diagonal table of
 * compiler/structural_lookups.py:279-333 to pairs.  Call with d_table = NULL
 * to get *entries_out (the sum of len^2, which must stay below 2^31), then
 * with buffers of n + 1 and `capacity` >= that many int32. */
int lcdhip_pair_lookup_build(const int32_t *d_ptr, const int32_t *d_idx, int64_t n,
                             int64_t idx_size, int32_t *d_base, int32_t *d_table,
                             int64_t capacity, int64_t *entries_out,
                             lcdhip_stream stream);

/* The same table with one byte per entry: the OFFSET of the found position
 * from the start of the segment searched (d_ptr[d_idx[d_ptr[s] + a]]), or -1;
 * every segment must have at most 127 entries (LCDHIP_ERR_ARGUMENT
 * otherwise).  A quarter of the bytes of lcdhip_pair_lookup_build for the
 * structures whose segments live in registers (at most 64 entries): on the
 * 9-point 1024^2 grid 81 MB instead of 324 MB, read once per factorization.
 * The caller adds the segment's start, which it has gathered by its own
 * positions (lcdhip_gather_i32 of d_ptr through d_idx).  Same reference
 * lines as above. */
int lcdhip_pair_offsets_build(const int32_t *d_ptr, const int32_t *d_idx, int64_t n,
                              int64_t idx_size, int32_t *d_base, int8_t *d_table,
                              int64_t capacity, int64_t *entries_out,
                              lcdhip_stream stream);

/* d_dst[q] = d_src[d_index[q] + offset] for q in [0, count): a structure
 * array read in the order the executor visits the tasks, so that a task's
 * loads of it (`Ap[i]`, `Ap[i + 1]`) have addresses that depend on the queue
 * position alone.  Fails with LCDHIP_ERR_ARGUMENT when an index leaves
 * [0, src_size).  (Layout of this backend's executors; the reference prefetches
 * the same node loads through the task id, compiler/cuda_lowering.py:1991-2029.) */
int lcdhip_gather_i32(int32_t *d_dst, const int32_t *d_src,
                      const int32_t *d_index, int64_t offset, int64_t count,
                      int64_t src_size, lcdhip_stream stream);

/* 128-bit content digest of a device array; replaces the per-call blake2b of
 * the structure arrays (compiler/scheduler.py:678-711) for arrays that are
 * already resident. */
int lcdhip_digest(const void *d_data, size_t bytes, uint64_t out[2],
                  lcdhip_stream stream);

/* The same digest for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc); it has no
 * counterpart in the reference.  Calls no hipMalloc/hipFree and does not
 * synchronise: two kernels are enqueued on `stream` and the 16-byte digest is
 * stored to the device buffer d_out[0..1], equal to what lcdhip_digest
 * returns for the same bytes.  The per-workgroup partial results go to a
 * 16 KiB work area inside the library, one per GPU, held until the process
 * ends and shared by every call on that GPU: calls that overlap on one GPU
 * (two streams) race.  bytes must be a multiple of 4 and at most
 * LCDHIP_DIGEST_NOALLOC_MAX_BYTES. */
#define LCDHIP_DIGEST_NOALLOC_MAX_BYTES ((size_t)1 << 36)
int lcdhip_digest_noalloc(const void *d_data, size_t bytes, uint64_t *d_out,
                          lcdhip_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* LCDHIP_H */

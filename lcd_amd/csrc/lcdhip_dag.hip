// On-device DAG inspector: edge enumeration with set semantics, unique
// in-degrees, edge multiplicities, CSR successors, level sets and the
// flattened wavefront arrays.  Replaces the generated Python `extract_dag`
// (compiler/dag_codegen.py:1151-1550) and compact_successors /
// wavefronts_from_dag / preprocess_wavefront
// (compiler/dag_preprocessing.py:115-204) of the reference.
//
// Bit-exactness with the reference comes from construction, not from atomics
// order: edges become 64-bit keys (src << 32 | dst) that are radix-sorted and
// made unique (a sorted set per source), counts are integer histograms, and
// the wavefront array is a stable sort of node ids by level.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include <rocprim/rocprim.hpp>

#include "lcdhip_common.h"

using lcdhip::resolve_stream;
using lcdhip::set_error;

struct lcdhip_dag {
    lcdhip_dag_info info{};
    int32_t *arrays[LCDHIP_DAG_ARRAYS] = {};
    int64_t counts[LCDHIP_DAG_ARRAYS] = {};
};

namespace {

constexpr int kBlock = 256;

// flags[0] endpoint / pointer out of range, flags[1] an edge with src >= dst
struct RuleDevice {
    const int32_t *ptr;
    const int32_t *idx;
    int64_t idx_size;
    int32_t owner_is_source;
    int32_t lower_offset;
    int32_t upper_offset;
    int32_t guard;
    int32_t break_at_owner;
};

__global__ void emit_keys_kernel(RuleDevice rule, int64_t n,
                                 unsigned long long *__restrict__ keys,
                                 int32_t *__restrict__ edge_count,
                                 int32_t *__restrict__ flags,
                                 unsigned long long *__restrict__ candidates)
{
    int64_t seg = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (seg >= n)
        return;
    int64_t lo = static_cast<int64_t>(rule.ptr[seg]) + rule.lower_offset;
    int64_t hi = static_cast<int64_t>(rule.ptr[seg + 1]) + rule.upper_offset;
    if (lo < hi && (lo < 0 || hi > rule.idx_size)) {
        flags[0] = 1;
        return;
    }
    unsigned long long hits = 0;
    for (int64_t p = lo; p < hi; ++p) {
        int64_t other = rule.idx[p];
        if (rule.break_at_owner && other >= seg)
            break;
        int64_t src = rule.owner_is_source ? seg : other;
        int64_t dst = rule.owner_is_source ? other : seg;
        if (rule.guard == LCDHIP_GUARD_GREATER && !(dst > src))
            continue;
        if (rule.guard == LCDHIP_GUARD_NOT_EQUAL && src == dst)
            continue;
        if (other < 0 || other >= n) {
            flags[0] = 1;
            continue;
        }
        if (src >= dst)
            flags[1] = 1;
        keys[p] = (static_cast<unsigned long long>(src) << 32) |
                  static_cast<unsigned long long>(dst);
        atomicAdd(&edge_count[dst], 1);
        ++hits;
    }
    if (hits)
        atomicAdd(candidates, hits);
}

// Relational rule: every task seg releases all tasks j >= seg + first.  One
// thread per (seg, j) pair; the key slot of the pair is its rank in (seg, j)
// order.
__device__ __host__ inline int64_t later_prefix(int64_t seg, int64_t span)
{
    // pairs emitted by tasks below seg; task t emits max(span - t, 0) pairs
    int64_t full = seg < span ? seg : span;
    return full * span - full * (full - 1) / 2;
}

__global__ void emit_later_keys_kernel(int64_t n, int32_t first,
                                       unsigned long long *__restrict__ keys,
                                       int32_t *__restrict__ edge_count,
                                       unsigned long long *__restrict__ candidates)
{
    int64_t seg = blockIdx.y;
    int64_t j = seg + first + blockIdx.x * static_cast<int64_t>(blockDim.x) +
                threadIdx.x;
    if (j >= n)
        return;
    int64_t slot = later_prefix(seg, n - first) + (j - seg - first);
    keys[slot] = (static_cast<unsigned long long>(seg) << 32) |
                 static_cast<unsigned long long>(j);
    atomicAdd(&edge_count[j], 1);
    if (j == seg + first)
        atomicAdd(candidates, static_cast<unsigned long long>(n - j));
}

// Chain rule: task seg releases task seg + step only (the transitive
// reduction of the complete order when step == 1).
__global__ void emit_next_keys_kernel(int64_t n, int32_t step,
                                      unsigned long long *__restrict__ keys,
                                      int32_t *__restrict__ edge_count,
                                      unsigned long long *__restrict__ candidates)
{
    int64_t seg = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (seg + step >= n)
        return;
    keys[seg] = (static_cast<unsigned long long>(seg) << 32) |
                static_cast<unsigned long long>(seg + step);
    atomicAdd(&edge_count[seg + step], 1);
    if (seg == 0)
        atomicAdd(candidates, static_cast<unsigned long long>(n - step));
}

// From the sorted unique keys: successor array, unique in-degree and the
// out-degree histogram (scanned into dag_ptr afterwards).
__global__ void split_edges_kernel(const unsigned long long *__restrict__ keys,
                                   int64_t edges,
                                   int32_t *__restrict__ out_degree,
                                   int32_t *__restrict__ dag_index,
                                   int32_t *__restrict__ dep_count,
                                   unsigned long long *__restrict__ transposed)
{
    int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (e >= edges)
        return;
    unsigned long long key = keys[e];
    int64_t src = static_cast<int64_t>(key >> 32);
    int32_t dst = static_cast<int32_t>(key & 0xffffffffull);
    dag_index[e] = dst;
    atomicAdd(&dep_count[dst], 1);
    atomicAdd(&out_degree[src], 1);
    if (transposed)
        transposed[e] = (static_cast<unsigned long long>(dst) << 32) |
                        static_cast<unsigned long long>(src);
}

// (dst << 32 | src) keys with their position for every valid candidate.
__global__ void incoming_keys_kernel(const unsigned long long *__restrict__ keys,
                                     int64_t capacity,
                                     unsigned long long *__restrict__ out_keys,
                                     int32_t *__restrict__ out_positions)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p >= capacity)
        return;
    unsigned long long key = keys[p];
    out_positions[p] = static_cast<int32_t>(p);
    out_keys[p] = key == ~0ull ? key : ((key << 32) | (key >> 32));
}

// out_slot[in_pos[k]] = k: the inverse of the incoming listing.
__global__ void out_slot_kernel(const int32_t *__restrict__ in_pos,
                                int64_t count, int32_t *__restrict__ out_slot)
{
    int64_t k = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (k < count)
        out_slot[in_pos[k]] = static_cast<int32_t>(k);
}


// ---- band chains: connected components inside bands of consecutive levels

__global__ void position_of_kernel(const int32_t *__restrict__ wavefronts,
                                   int64_t n, int32_t *__restrict__ position_of,
                                   int32_t *__restrict__ parent)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p >= n)
        return;
    position_of[wavefronts[p]] = static_cast<int32_t>(p);
    parent[p] = static_cast<int32_t>(p);
}

__device__ __forceinline__ int32_t chain_root(const int32_t *parent, int32_t p)
{
    // parents only ever decrease, so a stale read still leads to the root
    int32_t q = __hip_atomic_load(&parent[p], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
    while (q != p) {
        p = q;
        q = __hip_atomic_load(&parent[p], __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
    }
    return p;
}

// One pass over the edges whose endpoints share a band: the larger root is
// hung under the smaller one.  A hook can lose against a concurrent smaller
// one; the pass is repeated until no edge joins two roots.
__global__ void chain_hook_kernel(const int32_t *__restrict__ dag_ptr,
                                  const int32_t *__restrict__ dag_index,
                                  const int32_t *__restrict__ level_of,
                                  const int32_t *__restrict__ position_of,
                                  int64_t n, int32_t band_width,
                                  int32_t *parent, int32_t *changed)
{
    int64_t u = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (u >= n)
        return;
    const int32_t band = level_of[u] / band_width;
    const int32_t pu = position_of[u];
    for (int32_t e = dag_ptr[u]; e < dag_ptr[u + 1]; ++e) {
        const int32_t v = dag_index[e];
        if (level_of[v] / band_width != band)
            continue;
        int32_t a = chain_root(parent, pu);
        int32_t b = chain_root(parent, position_of[v]);
        if (a == b)
            continue;
        const int32_t high = a > b ? a : b, low = a > b ? b : a;
        atomicMin(&parent[high], low);
        *changed = 1;
    }
}

__global__ void chain_compress_kernel(int32_t *parent, int64_t n)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p < n)
        parent[p] = chain_root(parent, static_cast<int32_t>(p));
}

__global__ void chain_keys_kernel(const int32_t *__restrict__ parent, int64_t n,
                                  unsigned long long *__restrict__ keys)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p < n)
        keys[p] = (static_cast<unsigned long long>(parent[p]) << 32) |
                  static_cast<unsigned long long>(p);
}

// sorted keys (root position, member position) -> members, chain starts
__global__ void chain_members_kernel(const unsigned long long *__restrict__ keys,
                                     const int32_t *__restrict__ wavefronts,
                                     int64_t n, int32_t *__restrict__ task_nodes,
                                     int32_t *__restrict__ starts)
{
    int64_t k = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (k >= n)
        return;
    task_nodes[k] = wavefronts[keys[k] & 0xffffffffull];
    starts[k] = (k == 0 || (keys[k] >> 32) != (keys[k - 1] >> 32)) ? 1 : 0;
}

__global__ void chain_offsets_kernel(const unsigned long long *__restrict__ keys,
                                     const int32_t *__restrict__ starts,
                                     const int32_t *__restrict__ task_of,
                                     const int32_t *__restrict__ wavefronts,
                                     const int32_t *__restrict__ level_of,
                                     int64_t n, int32_t band_width,
                                     int32_t *__restrict__ task_ptr,
                                     int32_t *__restrict__ band_tasks)
{
    int64_t k = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (k >= n || !starts[k])
        return;
    task_ptr[task_of[k]] = static_cast<int32_t>(k);
    const int32_t first = wavefronts[keys[k] >> 32];
    atomicAdd(&band_tasks[level_of[first] / band_width], 1);
}

// edges whose endpoints fall into the same tile of tile_rows consecutive ids
__global__ void tile_local_edges_kernel(const int32_t *__restrict__ dag_ptr,
                                        const int32_t *__restrict__ dag_index,
                                        int64_t n, int32_t tile_rows,
                                        unsigned long long *local_edges)
{
    int64_t u = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    unsigned long long mine = 0;
    if (u < n) {
        const int32_t tile = static_cast<int32_t>(u / tile_rows);
        for (int32_t e = dag_ptr[u]; e < dag_ptr[u + 1]; ++e)
            mine += dag_index[e] / tile_rows == tile ? 1u : 0u;
    }
    for (int offset = 32; offset > 0; offset >>= 1)
        mine += __shfl_xor(mine, offset, 64);
    if ((threadIdx.x & 63) == 0 && mine)
        atomicAdd(local_edges, mine);
}

__global__ void tile_keys_kernel(const int32_t *__restrict__ wavefronts,
                                 int64_t n, int32_t tile_rows,
                                 uint32_t *__restrict__ keys)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p < n)
        keys[p] = static_cast<uint32_t>(wavefronts[p] / tile_rows);
}

// box of a structured grid that holds the node id = x + nx * (y + ny * z);
// boxes are numbered in (z, y, x) order
__global__ void box_keys_kernel(const int32_t *__restrict__ wavefronts,
                                int64_t n, int32_t nx, int32_t ny,
                                int32_t bx, int32_t by, int32_t bz,
                                int32_t boxes_x, int32_t boxes_y,
                                uint32_t *__restrict__ keys)
{
    int64_t p = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (p >= n)
        return;
    const int32_t id = wavefronts[p];
    const int32_t x = id % nx, rest = id / nx;
    const int32_t y = rest % ny, z = rest / ny;
    keys[p] = static_cast<uint32_t>(((z / bz) * boxes_y + y / by) * boxes_x +
                                    x / bx);
}

__global__ void inverse_order_kernel(const int32_t *__restrict__ order,
                                     int64_t n, int32_t *__restrict__ position)
{
    int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (q < n)
        position[order[q]] = static_cast<int32_t>(q);
}

// destination - source of every unique edge, biased so that unsigned order is
// signed order
__global__ void edge_offsets_kernel(const int32_t *__restrict__ dag_ptr,
                                    const int32_t *__restrict__ dag_index,
                                    int64_t n, uint32_t *__restrict__ offsets)
{
    int64_t u = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (u >= n)
        return;
    for (int32_t e = dag_ptr[u]; e < dag_ptr[u + 1]; ++e)
        offsets[e] = static_cast<uint32_t>(dag_index[e] - static_cast<int32_t>(u)) +
                     0x80000000u;
}

__global__ void low_words_kernel(const unsigned long long *__restrict__ keys,
                                 int64_t count, int32_t *__restrict__ out)
{
    int64_t e = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (e < count)
        out[e] = static_cast<int32_t>(keys[e] & 0xffffffffull);
}

__global__ void iota_kernel(int32_t *out, int64_t count)
{
    int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i < count)
        out[i] = static_cast<int32_t>(i);
}

// ---- level sets, algorithm 1: frontier expansion (Kahn) ------------------
// counts[0..2] rotating frontier sizes, counts[3] scheduled nodes,
// counts[4] number of levels.

__global__ void kahn_seed_kernel(const int32_t *__restrict__ dep_count,
                                 int64_t n, int32_t *__restrict__ frontier,
                                 int32_t *__restrict__ counts)
{
    int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (v < n && dep_count[v] == 0)
        frontier[atomicAdd(&counts[0], 1)] = static_cast<int32_t>(v);
}

__global__ void kahn_expand_kernel(const int32_t *__restrict__ dag_ptr,
                                   const int32_t *__restrict__ dag_index,
                                   int32_t *__restrict__ remaining,
                                   int32_t *__restrict__ level_of,
                                   const int32_t *__restrict__ current,
                                   int32_t *__restrict__ next,
                                   int32_t *__restrict__ counts, int32_t level)
{
    const int32_t size = counts[level % 3];
    int32_t *next_count = &counts[(level + 1) % 3];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        counts[(level + 2) % 3] = 0;
        if (size > 0) {
            atomicAdd(&counts[3], size);
            atomicMax(&counts[4], level + 1);
        }
    }
    int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t q = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
         q < size; q += stride) {
        int32_t v = current[q];
        level_of[v] = level;
        for (int32_t e = dag_ptr[v]; e < dag_ptr[v + 1]; ++e) {
            int32_t w = dag_index[e];
            if (atomicSub(&remaining[w], 1) == 1)
                next[atomicAdd(next_count, 1)] = w;
        }
    }
}

// ---- level sets, algorithm 2: ordered sweep ------------------------------
// Valid when every edge goes from a lower to a higher id.  Wavefronts take
// 64 consecutive ids in order, a lane per node; level(v) = 1 + max
// level(pred).  Predecessor lists are sorted, so a node's predecessors in
// earlier chunks come first and those inside its own chunk last.  The former
// are read from memory: once with a plain load (a level is written once over
// the -1 the array starts with, so any other value is final whichever cache
// served it), then, where that came back -1, with device-coherent polls and a
// nap between them.  The latter go through LDS alone: between two rounds of
// polls the chunk settles every chain among its own nodes that has become
// free, at LDS latency and with no load from memory in the way.  Chunks are
// handed out in id order, so the lowest unfinished chunk can always finish:
// no deadlock.  state[0] chunk counter, state[1] watchdog flag, state[2] max
// level + 1.
// Sum of (destination - source) over every kSpanSample-th edge of the
// (dst << 32 | src) keys: how far back a node's predecessors lie on average.
constexpr int kSpanSample = 16;

__global__ void edge_span_kernel(const unsigned long long *__restrict__ keys,
                                 int64_t edges, unsigned long long *sum)
{
    const int64_t e = (blockIdx.x * static_cast<int64_t>(blockDim.x) +
                       threadIdx.x) * kSpanSample;
    unsigned long long span = 0;
    if (e < edges) {
        const unsigned long long key = keys[e];
        span = (key >> 32) - (key & 0xffffffffull);
    }
    for (int offset = 32; offset > 0; offset >>= 1)
        span += __shfl_xor(span, offset);
    if ((threadIdx.x & 63) == 0 && span)
        atomicAdd(sum, span);
}

constexpr int32_t kHeavyNode = 96;   // predecessors beyond which the wavefront helps

__global__ void __launch_bounds__(256)
sweep_levels_kernel(const int32_t *__restrict__ pred_ptr,
                    const int32_t *__restrict__ pred_index, int64_t n,
                    int32_t *level_of, int32_t *state)
{
    __shared__ volatile int32_t chunk_level[4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int32_t highest = 0;
    while (true) {
        int32_t chunk = 0;
        if (lane == 0)
            chunk = atomicAdd(&state[0], 1);
        chunk = __shfl(chunk, 0);
        const int64_t base = static_cast<int64_t>(chunk) * 64;
        if (base >= n)
            break;
        const int64_t v = base + lane;
        bool pending = v < n;
        chunk_level[wave][lane] = -1;
        int32_t p = pending ? pred_ptr[v] : 0;
        const int32_t p_end = pending ? pred_ptr[v + 1] : 0;
        int32_t best = -1;
        // A node with many predecessors (a dense row of a power-law matrix)
        // is first read by the whole wavefront, 64 predecessors at a time:
        // the levels that are there already go into its maximum at once, and
        // its lane takes over at the first one that is still missing (they
        // are sorted, and what is missing is what was handed out last, so
        // that is near the end of the list).  Nobody waits here.
        unsigned long long heavy = __ballot(pending && p_end - p > kHeavyNode);
        while (heavy) {
            const int owner = __ffsll(static_cast<long long>(heavy)) - 1;
            heavy &= heavy - 1;
            const int32_t q0 = __shfl(p, owner), q1 = __shfl(p_end, owner);
            int32_t stop = q1, high = -1;
            for (int32_t q = q0 + lane; q < q1; q += 64) {
                const int64_t u = pred_index[q];
                int32_t l = -1;
                if (u < base) {
                    l = level_of[u];
                    if (l < 0)
                        l = __hip_atomic_load(&level_of[u], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
                }
                if (l < 0) {
                    stop = q;        // inside the chunk, or not there yet
                    break;
                }
                high = l > high ? l : high;
            }
            for (int offset = 32; offset > 0; offset >>= 1) {
                const int32_t other_high = __shfl_xor(high, offset);
                const int32_t other_stop = __shfl_xor(stop, offset);
                high = other_high > high ? other_high : high;
                stop = other_stop < stop ? other_stop : stop;
            }
            if (lane == owner) {
                best = high > best ? high : best;
                p = stop;
            }
        }
        // first pass over the predecessors in earlier chunks: plain loads.
        // `u` is the predecessor at p (read once, when p gets there).
        int64_t u = pending && p < p_end ? pred_index[p] : -1;
        bool outside = pending && p < p_end && u < base;
        while (outside) {
            const int32_t l = level_of[u];
            if (l < 0)
                break;
            best = l > best ? l : best;
            ++p;
            u = p < p_end ? pred_index[p] : -1;
            outside = p < p_end && u < base;
        }
        int64_t spins = 0;
        while (__ballot(pending)) {
            while (outside) {
                const int32_t l = __hip_atomic_load(
                    &level_of[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (l < 0)
                    break;
                best = l > best ? l : best;
                ++p;
                u = p < p_end ? pred_index[p] : -1;
                outside = p < p_end && u < base;
            }
            // the chains inside the chunk, as far as they are free
            bool moved = true;
            while (moved) {
                bool finished = false;
                if (pending && !outside) {
                    while (p < p_end) {
                        const int32_t l = chunk_level[wave][u - base];
                        if (l < 0)
                            break;
                        best = l > best ? l : best;
                        ++p;
                        u = p < p_end ? pred_index[p] : -1;
                    }
                    if (p == p_end) {
                        const int32_t mine = best + 1;
                        chunk_level[wave][lane] = mine;
                        __hip_atomic_store(&level_of[v], mine, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                        highest = mine + 1 > highest ? mine + 1 : highest;
                        pending = false;
                        finished = true;
                    }
                }
                moved = __ballot(finished) != 0;
            }
            // (a short nap while the wait is young -- a neighbour's level
            // is a hop away --, a longer one for the chunks far behind)
            if (__ballot(outside)) {
                if (spins < 16)
                    __builtin_amdgcn_s_sleep(1);
                else
                    __builtin_amdgcn_s_sleep(16);
            }
            // (every wait ends: a bound on the rounds of one chunk, and a
            // look at the flag another wavefront may have raised)
            if (++spins > (1ll << 22) ||
                ((spins & 255) == 0 &&
                 __hip_atomic_load(&state[1], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT))) {
                state[1] = 1;
                return;
            }
        }
    }
    for (int offset = 32; offset > 0; offset >>= 1) {
        int32_t other = __shfl_down(highest, offset);
        highest = other > highest ? other : highest;
    }
    if (lane == 0 && highest > 0)
        atomicMax(&state[2], highest);
}

// Shortcut of the ordered sweep for chains.  With ids in topological order
// level(v) <= v, and a node whose predecessors include v - 1 has
// level(v) >= level(v - 1) + 1; so on the longest prefix [0, m) in which every
// node v >= 1 has the predecessor v - 1 the level is the id itself.
// Predecessor lists are sorted, so v - 1 can only be the last entry.
// state[3] receives m (the host sets it to n beforehand).
__global__ void chain_prefix_kernel(const int32_t *__restrict__ pred_ptr,
                                    const int32_t *__restrict__ pred_index,
                                    int64_t n, int32_t *state)
{
    int64_t v = 1 + blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (v >= n)
        return;
    const int32_t end = pred_ptr[v + 1];
    if (end == pred_ptr[v] || pred_index[end - 1] != v - 1)
        atomicMin(&state[3], static_cast<int32_t>(v));
}

// level_of[v] = v on the chain prefix; the sweep's chunk counter starts at the
// chunk that holds the first node behind it.
__global__ void chain_fill_kernel(int64_t n, int32_t *__restrict__ level_of,
                                  int32_t *state)
{
    const int32_t m = state[3];
    int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (v == 0) {
        state[0] = m / 64;
        atomicMax(&state[2], m);
    }
    if (v < m)
        level_of[v] = static_cast<int32_t>(v);
}

// Nodes per level.  With few levels every bin is hot: a workgroup counts its
// share in LDS first (levels below kHistogramBins) and adds what it found to
// memory once per bin.
constexpr int kHistogramBins = 4096;

__global__ void __launch_bounds__(256)
level_histogram_kernel(const int32_t *__restrict__ level_of, int64_t n,
                       int32_t *__restrict__ hist)
{
    __shared__ int32_t bins[kHistogramBins];
    for (int b = threadIdx.x; b < kHistogramBins; b += blockDim.x)
        bins[b] = 0;
    __syncthreads();
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t v = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
         v < n; v += stride) {
        const int32_t level = level_of[v];
        if (level < 0)
            continue;
        if (level < kHistogramBins)
            atomicAdd(&bins[level], 1);
        else
            atomicAdd(&hist[level], 1);
    }
    __syncthreads();
    for (int b = threadIdx.x; b < kHistogramBins; b += blockDim.x)
        if (bins[b])
            atomicAdd(&hist[b], bins[b]);
}

inline unsigned blocks_for(int64_t count)
{
    return static_cast<unsigned>((count + kBlock - 1) / kBlock);
}

inline int bits_for(uint64_t max_value)
{
    int bits = 1;
    while (bits < 64 && (max_value >> bits))
        ++bits;
    return bits;
}

// Temporaries of one inspector call, from the library's block pool.  They go
// back when the call returns, behind one wait for the device: work that
// still reads them may be in flight (hipFree used to wait the same way).
struct Scratch {
    std::vector<void *> owned;
    ~Scratch()
    {
        lcdhip::pool_retire(owned.data(), owned.size());
    }
    template <class T>
    hipError_t alloc(T **out, size_t count)
    {
        void *p = nullptr;
        hipError_t status =
            lcdhip::pool_alloc(&p, std::max<size_t>(count, 1) * sizeof(T));
        if (status == hipSuccess)
            owned.push_back(p);
        *out = static_cast<T *>(p);
        return status;
    }
};

}  // namespace

extern "C" int lcdhip_dag_destroy(lcdhip_dag *dag)
{
    if (!dag)
        return LCDHIP_OK;
    // (the arrays may still be read by work in flight)
    void *blocks[LCDHIP_DAG_ARRAYS];
    for (int which = 0; which < LCDHIP_DAG_ARRAYS; ++which) {
        blocks[which] = dag->arrays[which];
        dag->arrays[which] = nullptr;
    }
    lcdhip::pool_retire(blocks, LCDHIP_DAG_ARRAYS);
    delete dag;
    return LCDHIP_OK;
}

static int dag_alloc(lcdhip_dag *dag, int which, int64_t count)
{
    void *block = nullptr;
    LCDHIP_CHECK(lcdhip::pool_alloc(
        &block, std::max<int64_t>(count, 1) * sizeof(int32_t)));
    dag->arrays[which] = static_cast<int32_t *>(block);
    dag->counts[which] = count;
    return LCDHIP_OK;
}

static int build_levels(lcdhip_dag *dag, const unsigned long long *d_transposed,
                        uint32_t flags, hipStream_t stream);

extern "C" int lcdhip_dag_build(const lcdhip_dag_rule *rules, int rule_count,
                                int64_t n, uint32_t flags, lcdhip_stream stream_,
                                lcdhip_dag **out)
{
    LCDHIP_REQUIRE_INIT();
    if (!out || rule_count < 0 || (rule_count > 0 && !rules) || n < 0 ||
        n >= (int64_t(1) << 31) - 1) {
        set_error("bad argument to lcdhip_dag_build");
        return LCDHIP_ERR_ARGUMENT;
    }
    *out = nullptr;
    hipStream_t stream = resolve_stream(stream_);
    int64_t key_capacity = 0;
    std::vector<int64_t> rule_keys(rule_count, 0);
    for (int r = 0; r < rule_count; ++r) {
        if (rules[r].relation == LCDHIP_RULE_LATER) {
            if (rules[r].lower_offset < 1 || n > 65535 ||
                (flags & LCDHIP_DAG_INCOMING)) {
                set_error("rule %d: a relational rule needs lower_offset >= 1,"
                          " at most 65535 tasks and no incoming listing", r);
                return LCDHIP_ERR_ARGUMENT;
            }
            int64_t span = std::max<int64_t>(n - rules[r].lower_offset, 0);
            rule_keys[r] = span * (span + 1) / 2;
        } else if (rules[r].relation == LCDHIP_RULE_NEXT) {
            if (rules[r].lower_offset < 1 || (flags & LCDHIP_DAG_INCOMING)) {
                set_error("rule %d: a chain rule needs lower_offset >= 1 and "
                          "no incoming listing", r);
                return LCDHIP_ERR_ARGUMENT;
            }
            rule_keys[r] = std::max<int64_t>(n - rules[r].lower_offset, 0);
        } else if (rules[r].relation != LCDHIP_RULE_SEGMENT) {
            set_error("rule %d has an unknown relation %d", r,
                      rules[r].relation);
            return LCDHIP_ERR_ARGUMENT;
        } else if (!rules[r].d_ptr || rules[r].idx_size < 0 ||
                   (rules[r].idx_size > 0 && !rules[r].d_idx)) {
            set_error("rule %d has a NULL structure array", r);
            return LCDHIP_ERR_ARGUMENT;
        } else {
            rule_keys[r] = rules[r].idx_size;
        }
        key_capacity += rule_keys[r];
    }
    if (key_capacity >= (int64_t(1) << 31)) {
        set_error("more than 2^31 candidate edges are not supported");
        return LCDHIP_ERR_ARGUMENT;
    }

    lcdhip_dag *dag = new lcdhip_dag();
    struct Guard {
        lcdhip_dag *dag;
        ~Guard() { if (dag) lcdhip_dag_destroy(dag); }
    } guard{dag};
    dag->info.n = n;
    int status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_PTR, n + 1))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_DEP_COUNT, n))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_EDGE_COUNT, n))) return status;
    int32_t *dag_ptr = dag->arrays[LCDHIP_DAG_PTR];
    int32_t *dep_count = dag->arrays[LCDHIP_DAG_DEP_COUNT];
    int32_t *edge_count = dag->arrays[LCDHIP_DAG_EDGE_COUNT];
    LCDHIP_CHECK(hipMemsetAsync(dag_ptr, 0, (n + 1) * 4, stream));
    LCDHIP_CHECK(hipMemsetAsync(dep_count, 0, std::max<int64_t>(n, 1) * 4, stream));
    LCDHIP_CHECK(hipMemsetAsync(edge_count, 0, std::max<int64_t>(n, 1) * 4, stream));

    Scratch scratch;
    unsigned long long *keys = nullptr, *sorted = nullptr, *unique_keys = nullptr;
    unsigned long long *d_candidates = nullptr;
    int32_t *d_flags = nullptr;
    LCDHIP_CHECK(scratch.alloc(&keys, key_capacity));
    LCDHIP_CHECK(scratch.alloc(&sorted, key_capacity));
    LCDHIP_CHECK(scratch.alloc(&d_candidates, 2));
    LCDHIP_CHECK(scratch.alloc(&d_flags, 4));
    LCDHIP_CHECK(hipMemsetAsync(keys, 0xff, std::max<int64_t>(key_capacity, 1) * 8, stream));
    LCDHIP_CHECK(hipMemsetAsync(d_candidates, 0, 16, stream));
    LCDHIP_CHECK(hipMemsetAsync(d_flags, 0, 16, stream));

    int64_t offset = 0;
    for (int r = 0; r < rule_count && n > 0; ++r) {
        if (rules[r].relation == LCDHIP_RULE_LATER) {
            if (rule_keys[r] > 0)
                hipLaunchKernelGGL(
                    emit_later_keys_kernel,
                    dim3(blocks_for(n - rules[r].lower_offset),
                         static_cast<unsigned>(n - rules[r].lower_offset)),
                    dim3(kBlock), 0, stream, n, rules[r].lower_offset,
                    keys + offset, edge_count, d_candidates);
            offset += rule_keys[r];
            continue;
        }
        if (rules[r].relation == LCDHIP_RULE_NEXT) {
            if (rule_keys[r] > 0)
                hipLaunchKernelGGL(emit_next_keys_kernel,
                                   dim3(blocks_for(rule_keys[r])), dim3(kBlock),
                                   0, stream, n, rules[r].lower_offset,
                                   keys + offset, edge_count, d_candidates);
            offset += rule_keys[r];
            continue;
        }
        RuleDevice rule{rules[r].d_ptr,         rules[r].d_idx,
                        rules[r].idx_size,      rules[r].owner_is_source,
                        rules[r].lower_offset,  rules[r].upper_offset,
                        rules[r].guard,         rules[r].break_at_owner};
        hipLaunchKernelGGL(emit_keys_kernel, dim3(blocks_for(n)), dim3(kBlock),
                           0, stream, rule, n, keys + offset, edge_count,
                           d_flags, d_candidates);
        offset += rule_keys[r];
    }
    LCDHIP_CHECK(hipGetLastError());
    unsigned long long candidates = 0;
    int32_t host_flags[4] = {0, 0, 0, 0};
    LCDHIP_CHECK(hipMemcpyAsync(&candidates, d_candidates, 8,
                                hipMemcpyDeviceToHost, stream));
    LCDHIP_CHECK(hipMemcpyAsync(host_flags, d_flags, 16, hipMemcpyDeviceToHost,
                                stream));
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    if (host_flags[0]) {
        set_error("a DAG edge endpoint or segment bound is out of range "
                  "[0, %lld)", static_cast<long long>(n));
        return LCDHIP_ERR_DAG_BOUNDS;
    }
    dag->info.topological_ids = host_flags[1] ? 0 : 1;

    if (flags & LCDHIP_DAG_INCOMING) {
        // in_ptr = scan of the multiplicities; in_pos = positions stably
        // sorted by (dst, src): ties keep ascending position
        if ((status = dag_alloc(dag, LCDHIP_DAG_IN_PTR, n + 1))) return status;
        if ((status = dag_alloc(dag, LCDHIP_DAG_IN_POS,
                                static_cast<int64_t>(candidates))))
            return status;
        if ((status = dag_alloc(dag, LCDHIP_DAG_OUT_SLOT, key_capacity)))
            return status;
        if ((status = dag_alloc(dag, LCDHIP_DAG_IN_SRC,
                                static_cast<int64_t>(candidates))))
            return status;
        if (key_capacity > 0)
            LCDHIP_CHECK(hipMemsetAsync(dag->arrays[LCDHIP_DAG_OUT_SLOT], 0xff,
                                        key_capacity * 4, stream));
        int32_t *in_ptr = dag->arrays[LCDHIP_DAG_IN_PTR];
        LCDHIP_CHECK(hipMemsetAsync(in_ptr, 0, (n + 1) * 4, stream));
        if (n > 0) {
            size_t scan_bytes = 0;
            char *scan_temp = nullptr;
            LCDHIP_CHECK(rocprim::exclusive_scan(
                nullptr, scan_bytes, edge_count, in_ptr, 0,
                static_cast<size_t>(n), rocprim::plus<int32_t>(), stream));
            LCDHIP_CHECK(scratch.alloc(&scan_temp, scan_bytes));
            LCDHIP_CHECK(rocprim::exclusive_scan(
                scan_temp, scan_bytes, edge_count, in_ptr, 0,
                static_cast<size_t>(n), rocprim::plus<int32_t>(), stream));
            int32_t total = static_cast<int32_t>(candidates);
            LCDHIP_CHECK(hipMemcpyAsync(in_ptr + n, &total, 4,
                                        hipMemcpyHostToDevice, stream));
            LCDHIP_CHECK(hipStreamSynchronize(stream));
        }
        if (candidates > 0) {
            unsigned long long *in_keys = nullptr, *in_sorted = nullptr;
            int32_t *positions = nullptr, *sorted_positions = nullptr;
            LCDHIP_CHECK(scratch.alloc(&in_keys, key_capacity));
            LCDHIP_CHECK(scratch.alloc(&in_sorted, key_capacity));
            LCDHIP_CHECK(scratch.alloc(&positions, key_capacity));
            LCDHIP_CHECK(scratch.alloc(&sorted_positions, key_capacity));
            hipLaunchKernelGGL(incoming_keys_kernel,
                               dim3(blocks_for(key_capacity)), dim3(kBlock), 0,
                               stream, keys, key_capacity, in_keys, positions);
            size_t sort_bytes = 0;
            char *sort_temp = nullptr;
            LCDHIP_CHECK(rocprim::radix_sort_pairs(
                nullptr, sort_bytes, in_keys, in_sorted, positions,
                sorted_positions, static_cast<size_t>(key_capacity), 0, 64,
                stream));
            LCDHIP_CHECK(scratch.alloc(&sort_temp, sort_bytes));
            LCDHIP_CHECK(rocprim::radix_sort_pairs(
                sort_temp, sort_bytes, in_keys, in_sorted, positions,
                sorted_positions, static_cast<size_t>(key_capacity), 0, 64,
                stream));
            LCDHIP_CHECK(hipMemcpyAsync(dag->arrays[LCDHIP_DAG_IN_POS],
                                        sorted_positions, candidates * 4,
                                        hipMemcpyDeviceToDevice, stream));
            // sorted keys are (dst << 32 | src): the low words are the sources
            hipLaunchKernelGGL(low_words_kernel,
                               dim3(blocks_for(static_cast<int64_t>(candidates))),
                               dim3(kBlock), 0, stream, in_sorted,
                               static_cast<int64_t>(candidates),
                               dag->arrays[LCDHIP_DAG_IN_SRC]);
            hipLaunchKernelGGL(out_slot_kernel,
                               dim3(blocks_for(static_cast<int64_t>(candidates))),
                               dim3(kBlock), 0, stream,
                               dag->arrays[LCDHIP_DAG_IN_POS],
                               static_cast<int64_t>(candidates),
                               dag->arrays[LCDHIP_DAG_OUT_SLOT]);
            LCDHIP_CHECK(hipGetLastError());
            LCDHIP_CHECK(hipStreamSynchronize(stream));
        }
    }

    // sorted set of (src, dst) pairs
    int64_t edges = 0;
    if (candidates > 0) {
        const int end_bit = std::min(64, 32 + bits_for(static_cast<uint64_t>(n)));
        size_t temp_bytes = 0;
        void *temp = nullptr;
        // invalid keys are all ones: they stay last under any bit window
        // that covers every valid key
        LCDHIP_CHECK(rocprim::radix_sort_keys(nullptr, temp_bytes, keys, sorted,
                                              static_cast<size_t>(key_capacity),
                                              0, end_bit, stream));
        LCDHIP_CHECK(scratch.alloc(reinterpret_cast<char **>(&temp), temp_bytes));
        LCDHIP_CHECK(rocprim::radix_sort_keys(temp, temp_bytes, keys, sorted,
                                              static_cast<size_t>(key_capacity),
                                              0, end_bit, stream));
        LCDHIP_CHECK(scratch.alloc(&unique_keys, candidates));
        size_t unique_temp_bytes = 0;
        void *unique_temp = nullptr;
        LCDHIP_CHECK(rocprim::unique(nullptr, unique_temp_bytes, sorted,
                                     unique_keys, d_candidates + 1,
                                     static_cast<size_t>(candidates),
                                     rocprim::equal_to<unsigned long long>(),
                                     stream));
        LCDHIP_CHECK(scratch.alloc(reinterpret_cast<char **>(&unique_temp),
                                   unique_temp_bytes));
        LCDHIP_CHECK(rocprim::unique(unique_temp, unique_temp_bytes, sorted,
                                     unique_keys, d_candidates + 1,
                                     static_cast<size_t>(candidates),
                                     rocprim::equal_to<unsigned long long>(),
                                     stream));
        unsigned long long unique_count = 0;
        LCDHIP_CHECK(hipMemcpyAsync(&unique_count, d_candidates + 1, 8,
                                    hipMemcpyDeviceToHost, stream));
        LCDHIP_CHECK(hipStreamSynchronize(stream));
        edges = static_cast<int64_t>(unique_count);
    }
    dag->info.edges = edges;
    if ((status = dag_alloc(dag, LCDHIP_DAG_INDEX, edges))) return status;

    const bool want_levels = flags & LCDHIP_DAG_LEVELS;
    const bool sweep = want_levels && dag->info.topological_ids &&
                       !(flags & LCDHIP_DAG_FORCE_KAHN);
    unsigned long long *transposed = nullptr;
    if (sweep && edges > 0)
        LCDHIP_CHECK(scratch.alloc(&transposed, edges));
    if (edges > 0) {
        int32_t *out_degree = nullptr;
        LCDHIP_CHECK(scratch.alloc(&out_degree, n + 1));
        LCDHIP_CHECK(hipMemsetAsync(out_degree, 0, (n + 1) * 4, stream));
        hipLaunchKernelGGL(split_edges_kernel, dim3(blocks_for(edges)),
                           dim3(kBlock), 0, stream, unique_keys, edges,
                           out_degree, dag->arrays[LCDHIP_DAG_INDEX], dep_count,
                           transposed);
        LCDHIP_CHECK(hipGetLastError());
        size_t scan_bytes = 0;
        char *scan_temp = nullptr;
        LCDHIP_CHECK(rocprim::exclusive_scan(
            nullptr, scan_bytes, out_degree, dag_ptr, 0,
            static_cast<size_t>(n + 1), rocprim::plus<int32_t>(), stream));
        LCDHIP_CHECK(scratch.alloc(&scan_temp, scan_bytes));
        LCDHIP_CHECK(rocprim::exclusive_scan(
            scan_temp, scan_bytes, out_degree, dag_ptr, 0,
            static_cast<size_t>(n + 1), rocprim::plus<int32_t>(), stream));
    }
    if (want_levels) {
        // the forward keys are no longer needed: release them before the
        // level pass allocates its own scratch
        status = build_levels(dag, transposed, flags, stream);
        if (status)
            return status;
    }
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    guard.dag = nullptr;
    *out = dag;
    return LCDHIP_OK;
}

static int build_levels(lcdhip_dag *dag, const unsigned long long *d_transposed,
                        uint32_t flags, hipStream_t stream)
{
    const int64_t n = dag->info.n, edges = dag->info.edges;
    int status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_LEVEL_OF, n))) return status;
    int32_t *level_of = dag->arrays[LCDHIP_DAG_LEVEL_OF];
    LCDHIP_CHECK(hipMemsetAsync(level_of, 0xff, std::max<int64_t>(n, 1) * 4, stream));
    const int32_t *dag_ptr = dag->arrays[LCDHIP_DAG_PTR];
    const int32_t *dag_index = dag->arrays[LCDHIP_DAG_INDEX];
    const int32_t *dep_count = dag->arrays[LCDHIP_DAG_DEP_COUNT];
    Scratch scratch;
    int64_t levels = 0, scheduled = 0;
    const bool sweep = dag->info.topological_ids &&
                       !(flags & LCDHIP_DAG_FORCE_KAHN);

    if (n == 0) {
        dag->info.level_algorithm = 0;
    } else if (sweep) {
        dag->info.level_algorithm = 2;
        // predecessor CSR: offsets are the scan of the unique in-degree
        int32_t *pred_ptr = nullptr, *pred_index = nullptr, *state = nullptr;
        LCDHIP_CHECK(scratch.alloc(&pred_ptr, n + 1));
        LCDHIP_CHECK(scratch.alloc(&pred_index, edges));
        LCDHIP_CHECK(scratch.alloc(&state, 4));
        LCDHIP_CHECK(hipMemsetAsync(state, 0, 16, stream));
        unsigned long long *span_sum = nullptr, host_span = 0;
        {
            size_t temp_bytes = 0;
            char *temp = nullptr;
            LCDHIP_CHECK(hipMemsetAsync(pred_ptr + n, 0, 4, stream));
            LCDHIP_CHECK(rocprim::exclusive_scan(
                nullptr, temp_bytes, dep_count, pred_ptr, 0,
                static_cast<size_t>(n), rocprim::plus<int32_t>(), stream));
            LCDHIP_CHECK(scratch.alloc(&temp, temp_bytes));
            LCDHIP_CHECK(rocprim::exclusive_scan(
                temp, temp_bytes, dep_count, pred_ptr, 0,
                static_cast<size_t>(n), rocprim::plus<int32_t>(), stream));
            int32_t total = static_cast<int32_t>(edges);
            LCDHIP_CHECK(hipMemcpyAsync(pred_ptr + n, &total, 4,
                                        hipMemcpyHostToDevice, stream));
            if (edges > 0) {
                LCDHIP_CHECK(scratch.alloc(&span_sum, 1));
                LCDHIP_CHECK(hipMemsetAsync(span_sum, 0, 8, stream));
                hipLaunchKernelGGL(
                    edge_span_kernel,
                    dim3(blocks_for((edges + kSpanSample - 1) / kSpanSample)),
                    dim3(kBlock), 0, stream, d_transposed, edges, span_sum);
                LCDHIP_CHECK(hipMemcpyAsync(&host_span, span_sum, 8,
                                            hipMemcpyDeviceToHost, stream));
            }
            LCDHIP_CHECK(hipStreamSynchronize(stream));
        }
        if (edges > 0) {
            unsigned long long *sorted = nullptr;
            LCDHIP_CHECK(scratch.alloc(&sorted, edges));
            size_t temp_bytes = 0;
            char *temp = nullptr;
            const int end_bit =
                std::min(64, 32 + bits_for(static_cast<uint64_t>(n)));
            LCDHIP_CHECK(rocprim::radix_sort_keys(
                nullptr, temp_bytes, d_transposed, sorted,
                static_cast<size_t>(edges), 0, end_bit, stream));
            LCDHIP_CHECK(scratch.alloc(&temp, temp_bytes));
            LCDHIP_CHECK(rocprim::radix_sort_keys(
                temp, temp_bytes, d_transposed, sorted,
                static_cast<size_t>(edges), 0, end_bit, stream));
            hipLaunchKernelGGL(low_words_kernel, dim3(blocks_for(edges)),
                               dim3(kBlock), 0, stream, sorted, edges,
                               pred_index);
        }
        // chain prefix: its levels are known without sweeping (`whole` stays
        // alive until the synchronisation behind the sweep)
        const int32_t whole = static_cast<int32_t>(n);
        LCDHIP_CHECK(hipMemcpyAsync(state + 3, &whole, 4, hipMemcpyHostToDevice,
                                    stream));
        if (n > 1)
            hipLaunchKernelGGL(chain_prefix_kernel, dim3(blocks_for(n - 1)),
                               dim3(kBlock), 0, stream, pred_ptr, pred_index, n,
                               state);
        hipLaunchKernelGGL(chain_fill_kernel, dim3(blocks_for(n)), dim3(kBlock),
                           0, stream, n, level_of, state);
        const int64_t chunks = (n + 63) / 64;
        // How many chunks are in flight at once.  The chunks wait for one
        // another through memory polls, and polls that cannot succeed yet
        // slow down the ones that can.  Predecessors that lie close (grids,
        // bands) are always among the chunks in flight: a wide window (four
        // workgroups per CU) gives the diagonal front of such a DAG its
        // parallelism (whole inspection of the 128^3 grid: 8.4 / 6.0 / 4.7 /
        // 4.7 ms at 1 / 2 / 4 / 8 per CU; of the 9-point 1024^2 ILU0 DAG,
        // 3070 levels deep: 8.4 / 6.9 / 6.9 / 7.7 ms).  Predecessors spread
        // over all earlier ids (a random or power-law matrix) are mostly
        // finished already under a narrow window (one workgroup per CU) and
        // mostly polled in vain under a wide one (1 M rows, 16 M edges, mean
        // span 0.25 n: the sweep alone 2.3 ms against 8.4 ms).
        const double mean_span =
            edges > 0 ? static_cast<double>(host_span) * kSpanSample /
                            static_cast<double>(edges)
                      : 0.0;
        const int per_cu = mean_span * 8.0 > static_cast<double>(n) ? 1 : 4;
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(
            (chunks + 3) / 4,
            static_cast<int64_t>(lcdhip::context().props.multiProcessorCount) *
                per_cu));
        hipLaunchKernelGGL(sweep_levels_kernel, dim3(blocks), dim3(256), 0,
                           stream, pred_ptr, pred_index, n, level_of, state);
        LCDHIP_CHECK(hipGetLastError());
        int32_t host_state[4] = {0, 0, 0, 0};
        LCDHIP_CHECK(hipMemcpyAsync(host_state, state, 16, hipMemcpyDeviceToHost,
                                    stream));
        LCDHIP_CHECK(hipStreamSynchronize(stream));
        if (host_state[1]) {
            set_error("the ordered level sweep gave up waiting");
            return LCDHIP_ERR_WATCHDOG;
        }
        levels = host_state[2];
        scheduled = n;
    } else {
        dag->info.level_algorithm = 1;
        int32_t *remaining = nullptr, *frontier_a = nullptr, *frontier_b = nullptr;
        int32_t *frontier_c = nullptr, *counts = nullptr;
        LCDHIP_CHECK(scratch.alloc(&remaining, n));
        LCDHIP_CHECK(scratch.alloc(&frontier_a, n));
        LCDHIP_CHECK(scratch.alloc(&frontier_b, n));
        LCDHIP_CHECK(scratch.alloc(&frontier_c, n));
        LCDHIP_CHECK(scratch.alloc(&counts, 8));
        LCDHIP_CHECK(hipMemcpyAsync(remaining, dep_count, n * 4,
                                    hipMemcpyDeviceToDevice, stream));
        LCDHIP_CHECK(hipMemsetAsync(counts, 0, 32, stream));
        hipLaunchKernelGGL(kahn_seed_kernel, dim3(blocks_for(n)), dim3(kBlock),
                           0, stream, dep_count, n, frontier_a, counts);
        int32_t *frontiers[3] = {frontier_a, frontier_b, frontier_c};
        const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(
            blocks_for(n),
            static_cast<int64_t>(lcdhip::context().props.multiProcessorCount) * 4));
        int32_t level = 0;
        int32_t host_counts[8];
        while (true) {
            const int batch = 32;
            for (int step = 0; step < batch; ++step, ++level)
                hipLaunchKernelGGL(kahn_expand_kernel, dim3(blocks),
                                   dim3(kBlock), 0, stream, dag_ptr, dag_index,
                                   remaining, level_of, frontiers[level % 3],
                                   frontiers[(level + 1) % 3], counts, level);
            LCDHIP_CHECK(hipGetLastError());
            LCDHIP_CHECK(hipMemcpyAsync(host_counts, counts, 32,
                                        hipMemcpyDeviceToHost, stream));
            LCDHIP_CHECK(hipStreamSynchronize(stream));
            if (host_counts[level % 3] == 0 || level > n + batch)
                break;
        }
        levels = host_counts[4];
        scheduled = host_counts[3];
    }
    dag->info.levels = levels;
    dag->info.scheduled = scheduled;

    // wavefront_ptr = exclusive scan of the level histogram; wavefronts =
    // node ids stably sorted by level (ascending id inside a level)
    if ((status = dag_alloc(dag, LCDHIP_DAG_WAVEFRONT_PTR, levels + 1))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_WAVEFRONTS, scheduled))) return status;
    int32_t *wavefront_ptr = dag->arrays[LCDHIP_DAG_WAVEFRONT_PTR];
    LCDHIP_CHECK(hipMemsetAsync(wavefront_ptr, 0, (levels + 1) * 4, stream));
    if (n > 0 && levels > 0) {
        int32_t *hist = nullptr;
        LCDHIP_CHECK(scratch.alloc(&hist, levels + 1));
        LCDHIP_CHECK(hipMemsetAsync(hist, 0, (levels + 1) * 4, stream));
        hipLaunchKernelGGL(
            level_histogram_kernel,
            dim3(std::min<unsigned>(
                blocks_for(n),
                static_cast<unsigned>(
                    lcdhip::context().props.multiProcessorCount) * 4)),
            dim3(256), 0, stream, level_of, n, hist);
        size_t temp_bytes = 0;
        char *temp = nullptr;
        LCDHIP_CHECK(rocprim::exclusive_scan(
            nullptr, temp_bytes, hist, wavefront_ptr, 0,
            static_cast<size_t>(levels + 1), rocprim::plus<int32_t>(), stream));
        LCDHIP_CHECK(scratch.alloc(&temp, temp_bytes));
        LCDHIP_CHECK(rocprim::exclusive_scan(
            temp, temp_bytes, hist, wavefront_ptr, 0,
            static_cast<size_t>(levels + 1), rocprim::plus<int32_t>(), stream));

        int32_t *ids = nullptr, *sorted_ids = nullptr;
        uint32_t *sorted_levels = nullptr;
        LCDHIP_CHECK(scratch.alloc(&ids, n));
        LCDHIP_CHECK(scratch.alloc(&sorted_ids, n));
        LCDHIP_CHECK(scratch.alloc(&sorted_levels, n));
        hipLaunchKernelGGL(iota_kernel, dim3(blocks_for(n)), dim3(kBlock), 0,
                           stream, ids, n);
        // unscheduled nodes carry level -1 = 0xffffffff and sort last
        const int end_bit = scheduled == n ? bits_for(static_cast<uint64_t>(levels)) : 32;
        size_t sort_bytes = 0;
        char *sort_temp = nullptr;
        LCDHIP_CHECK(rocprim::radix_sort_pairs(
            nullptr, sort_bytes, reinterpret_cast<const uint32_t *>(level_of),
            sorted_levels, ids, sorted_ids, static_cast<size_t>(n), 0, end_bit,
            stream));
        LCDHIP_CHECK(scratch.alloc(&sort_temp, sort_bytes));
        LCDHIP_CHECK(rocprim::radix_sort_pairs(
            sort_temp, sort_bytes, reinterpret_cast<const uint32_t *>(level_of),
            sorted_levels, ids, sorted_ids, static_cast<size_t>(n), 0, end_bit,
            stream));
        LCDHIP_CHECK(hipMemcpyAsync(dag->arrays[LCDHIP_DAG_WAVEFRONTS],
                                    sorted_ids, scheduled * 4,
                                    hipMemcpyDeviceToDevice, stream));
        std::vector<int32_t> host_ptr(levels + 1);
        LCDHIP_CHECK(hipMemcpyAsync(host_ptr.data(), wavefront_ptr,
                                    (levels + 1) * 4, hipMemcpyDeviceToHost,
                                    stream));
        LCDHIP_CHECK(hipStreamSynchronize(stream));
        int64_t widest = 0;
        for (int64_t l = 0; l < levels; ++l)
            widest = std::max<int64_t>(widest, host_ptr[l + 1] - host_ptr[l]);
        dag->info.max_level_width = widest;
    }
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    return LCDHIP_OK;
}

extern "C" int lcdhip_dag_band_chains(lcdhip_dag *dag, int64_t band_width,
                                      lcdhip_stream stream_handle,
                                      int64_t *tasks_out, int64_t *bands_out)
{
    LCDHIP_REQUIRE_INIT();
    if (!dag || band_width <= 0 || band_width > 0x7fffffff) {
        set_error("The band width must be a positive integer.");
        return LCDHIP_ERR_ARGUMENT;
    }
    if (!dag->arrays[LCDHIP_DAG_WAVEFRONTS] ||
        dag->info.scheduled != dag->info.n) {
        set_error("band chains need level sets that cover every node");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t stream = resolve_stream(stream_handle);
    const int64_t n = dag->info.n;
    const int64_t bands = (dag->info.levels + band_width - 1) / band_width;
    for (int which : {LCDHIP_DAG_TASK_NODES, LCDHIP_DAG_TASK_PTR,
                      LCDHIP_DAG_BAND_PTR})
        if (dag->arrays[which]) {
            void *block = dag->arrays[which];
            lcdhip::pool_retire(&block, 1);
            dag->arrays[which] = nullptr;
            dag->counts[which] = 0;
        }
    int status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_TASK_NODES, n))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_BAND_PTR, bands + 1))) return status;
    int32_t *band_ptr = dag->arrays[LCDHIP_DAG_BAND_PTR];
    LCDHIP_CHECK(hipMemsetAsync(band_ptr, 0, (bands + 1) * 4, stream));
    int64_t tasks = 0;
    if (n > 0) {
        const int32_t *wavefronts = dag->arrays[LCDHIP_DAG_WAVEFRONTS];
        const int32_t *level_of = dag->arrays[LCDHIP_DAG_LEVEL_OF];
        Scratch scratch;
        int32_t *position_of = nullptr, *parent = nullptr, *changed = nullptr;
        int32_t *starts = nullptr, *task_of = nullptr, *band_tasks = nullptr;
        unsigned long long *keys = nullptr, *sorted = nullptr;
        LCDHIP_CHECK(scratch.alloc(&position_of, n));
        LCDHIP_CHECK(scratch.alloc(&parent, n));
        LCDHIP_CHECK(scratch.alloc(&changed, 1));
        LCDHIP_CHECK(scratch.alloc(&starts, n));
        LCDHIP_CHECK(scratch.alloc(&task_of, n));
        LCDHIP_CHECK(scratch.alloc(&band_tasks, bands + 1));
        LCDHIP_CHECK(scratch.alloc(&keys, n));
        LCDHIP_CHECK(scratch.alloc(&sorted, n));
        hipLaunchKernelGGL(position_of_kernel, dim3(blocks_for(n)), dim3(kBlock),
                           0, stream, wavefronts, n, position_of, parent);
        // every pass at least halves nothing in the worst case, so bound the
        // passes by the node count; practical inputs need a handful
        for (int64_t pass = 0; pass <= n; ++pass) {
            int32_t flag = 0;
            LCDHIP_CHECK(hipMemsetAsync(changed, 0, 4, stream));
            hipLaunchKernelGGL(chain_hook_kernel, dim3(blocks_for(n)),
                               dim3(kBlock), 0, stream,
                               dag->arrays[LCDHIP_DAG_PTR],
                               dag->arrays[LCDHIP_DAG_INDEX], level_of,
                               position_of, n, static_cast<int32_t>(band_width),
                               parent, changed);
            hipLaunchKernelGGL(chain_compress_kernel, dim3(blocks_for(n)),
                               dim3(kBlock), 0, stream, parent, n);
            LCDHIP_CHECK(hipMemcpyAsync(&flag, changed, 4,
                                        hipMemcpyDeviceToHost, stream));
            LCDHIP_CHECK(hipStreamSynchronize(stream));
            if (!flag)
                break;
        }
        hipLaunchKernelGGL(chain_keys_kernel, dim3(blocks_for(n)), dim3(kBlock),
                           0, stream, parent, n, keys);
        const int end_bit = std::min(64, 32 + bits_for(static_cast<uint64_t>(n)));
        size_t sort_bytes = 0;
        char *sort_temp = nullptr;
        LCDHIP_CHECK(rocprim::radix_sort_keys(nullptr, sort_bytes, keys, sorted,
                                              static_cast<size_t>(n), 0, end_bit,
                                              stream));
        LCDHIP_CHECK(scratch.alloc(&sort_temp, sort_bytes));
        LCDHIP_CHECK(rocprim::radix_sort_keys(sort_temp, sort_bytes, keys, sorted,
                                              static_cast<size_t>(n), 0, end_bit,
                                              stream));
        hipLaunchKernelGGL(chain_members_kernel, dim3(blocks_for(n)),
                           dim3(kBlock), 0, stream, sorted, wavefronts, n,
                           dag->arrays[LCDHIP_DAG_TASK_NODES], starts);
        size_t scan_bytes = 0;
        char *scan_temp = nullptr;
        LCDHIP_CHECK(rocprim::exclusive_scan(nullptr, scan_bytes, starts, task_of,
                                             0, static_cast<size_t>(n),
                                             rocprim::plus<int32_t>(), stream));
        LCDHIP_CHECK(scratch.alloc(&scan_temp, scan_bytes));
        LCDHIP_CHECK(rocprim::exclusive_scan(scan_temp, scan_bytes, starts,
                                             task_of, 0, static_cast<size_t>(n),
                                             rocprim::plus<int32_t>(), stream));
        int32_t last_task = 0, last_start = 0;
        LCDHIP_CHECK(hipMemcpyAsync(&last_task, task_of + (n - 1), 4,
                                    hipMemcpyDeviceToHost, stream));
        LCDHIP_CHECK(hipMemcpyAsync(&last_start, starts + (n - 1), 4,
                                    hipMemcpyDeviceToHost, stream));
        LCDHIP_CHECK(hipStreamSynchronize(stream));
        tasks = static_cast<int64_t>(last_task) + last_start;
        if ((status = dag_alloc(dag, LCDHIP_DAG_TASK_PTR, tasks + 1)))
            return status;
        int32_t *task_ptr = dag->arrays[LCDHIP_DAG_TASK_PTR];
        LCDHIP_CHECK(hipMemsetAsync(band_tasks, 0, (bands + 1) * 4, stream));
        hipLaunchKernelGGL(chain_offsets_kernel, dim3(blocks_for(n)),
                           dim3(kBlock), 0, stream, sorted, starts, task_of,
                           wavefronts, level_of, n,
                           static_cast<int32_t>(band_width), task_ptr,
                           band_tasks);
        const int32_t total = static_cast<int32_t>(n);
        LCDHIP_CHECK(hipMemcpyAsync(task_ptr + tasks, &total, 4,
                                    hipMemcpyHostToDevice, stream));
        size_t band_bytes = 0;
        char *band_temp = nullptr;
        LCDHIP_CHECK(rocprim::exclusive_scan(
            nullptr, band_bytes, band_tasks, band_ptr, 0,
            static_cast<size_t>(bands + 1), rocprim::plus<int32_t>(), stream));
        LCDHIP_CHECK(scratch.alloc(&band_temp, band_bytes));
        LCDHIP_CHECK(rocprim::exclusive_scan(
            band_temp, band_bytes, band_tasks, band_ptr, 0,
            static_cast<size_t>(bands + 1), rocprim::plus<int32_t>(), stream));
        LCDHIP_CHECK(hipGetLastError());
        LCDHIP_CHECK(hipStreamSynchronize(stream));
    } else {
        if ((status = dag_alloc(dag, LCDHIP_DAG_TASK_PTR, 1))) return status;
        LCDHIP_CHECK(hipMemsetAsync(dag->arrays[LCDHIP_DAG_TASK_PTR], 0, 4,
                                    stream));
        LCDHIP_CHECK(hipStreamSynchronize(stream));
    }
    if (tasks_out)
        *tasks_out = tasks;
    if (bands_out)
        *bands_out = bands;
    return LCDHIP_OK;
}

extern "C" int lcdhip_dag_tile_locality(const lcdhip_dag *dag, int64_t tile_rows,
                                        lcdhip_stream stream_handle,
                                        int64_t *local_edges_out)
{
    LCDHIP_REQUIRE_INIT();
    if (!dag || !local_edges_out || tile_rows <= 0 || tile_rows > 0x7fffffff) {
        set_error("bad argument to lcdhip_dag_tile_locality");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t stream = resolve_stream(stream_handle);
    const int64_t n = dag->info.n;
    *local_edges_out = 0;
    if (n == 0 || dag->info.edges == 0)
        return LCDHIP_OK;
    Scratch scratch;
    unsigned long long *d_count = nullptr, host_count = 0;
    LCDHIP_CHECK(scratch.alloc(&d_count, 1));
    LCDHIP_CHECK(hipMemsetAsync(d_count, 0, 8, stream));
    hipLaunchKernelGGL(tile_local_edges_kernel, dim3(blocks_for(n)),
                       dim3(kBlock), 0, stream, dag->arrays[LCDHIP_DAG_PTR],
                       dag->arrays[LCDHIP_DAG_INDEX], n,
                       static_cast<int32_t>(tile_rows), d_count);
    LCDHIP_CHECK(hipGetLastError());
    LCDHIP_CHECK(hipMemcpyAsync(&host_count, d_count, 8, hipMemcpyDeviceToHost,
                                stream));
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    *local_edges_out = static_cast<int64_t>(host_count);
    return LCDHIP_OK;
}

namespace {

void dag_release(lcdhip_dag *dag, int which)
{
    if (dag->arrays[which]) {
        void *block = dag->arrays[which];
        lcdhip::pool_retire(&block, 1);
        dag->arrays[which] = nullptr;
        dag->counts[which] = 0;
    }
}

// TILE_NODES = the level-ordered node list sorted (stably) by `keys`, one key
// per position of WAVEFRONTS; TILE_POS = its inverse.
int tile_order_from_keys(lcdhip_dag *dag, Scratch &scratch, uint32_t *keys,
                         uint64_t key_count, hipStream_t stream)
{
    const int64_t n = dag->info.n;
    int status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_TILE_NODES, n))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_TILE_POS, n))) return status;
    uint32_t *sorted_keys = nullptr;
    LCDHIP_CHECK(scratch.alloc(&sorted_keys, n));
    // stable: inside a tile the (level, id) order of the level sets stays
    const int end_bit = bits_for(key_count);
    size_t sort_bytes = 0;
    char *sort_temp = nullptr;
    LCDHIP_CHECK(rocprim::radix_sort_pairs(
        nullptr, sort_bytes, keys, sorted_keys,
        dag->arrays[LCDHIP_DAG_WAVEFRONTS], dag->arrays[LCDHIP_DAG_TILE_NODES],
        static_cast<size_t>(n), 0, end_bit, stream));
    LCDHIP_CHECK(scratch.alloc(&sort_temp, sort_bytes));
    LCDHIP_CHECK(rocprim::radix_sort_pairs(
        sort_temp, sort_bytes, keys, sorted_keys,
        dag->arrays[LCDHIP_DAG_WAVEFRONTS], dag->arrays[LCDHIP_DAG_TILE_NODES],
        static_cast<size_t>(n), 0, end_bit, stream));
    hipLaunchKernelGGL(inverse_order_kernel, dim3(blocks_for(n)), dim3(kBlock),
                       0, stream, dag->arrays[LCDHIP_DAG_TILE_NODES], n,
                       dag->arrays[LCDHIP_DAG_TILE_POS]);
    LCDHIP_CHECK(hipGetLastError());
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    return LCDHIP_OK;
}

int tile_order_ready(lcdhip_dag *dag)
{
    if (!dag->arrays[LCDHIP_DAG_WAVEFRONTS] ||
        dag->info.scheduled != dag->info.n) {
        set_error("tiles need level sets that cover every node");
        return LCDHIP_ERR_ARGUMENT;
    }
    dag_release(dag, LCDHIP_DAG_TILE_NODES);
    dag_release(dag, LCDHIP_DAG_TILE_POS);
    return LCDHIP_OK;
}

}

extern "C" int lcdhip_dag_tile_order(lcdhip_dag *dag, int64_t tile_rows,
                                     lcdhip_stream stream_handle)
{
    LCDHIP_REQUIRE_INIT();
    if (!dag || tile_rows <= 0 || tile_rows > 0x7fffffff) {
        set_error("The tile size must be a positive integer.");
        return LCDHIP_ERR_ARGUMENT;
    }
    int status;
    if ((status = tile_order_ready(dag))) return status;
    hipStream_t stream = resolve_stream(stream_handle);
    const int64_t n = dag->info.n;
    if (n == 0) {
        if ((status = dag_alloc(dag, LCDHIP_DAG_TILE_NODES, 0))) return status;
        return dag_alloc(dag, LCDHIP_DAG_TILE_POS, 0);
    }
    Scratch scratch;
    uint32_t *keys = nullptr;
    LCDHIP_CHECK(scratch.alloc(&keys, n));
    hipLaunchKernelGGL(tile_keys_kernel, dim3(blocks_for(n)), dim3(kBlock), 0,
                       stream, dag->arrays[LCDHIP_DAG_WAVEFRONTS], n,
                       static_cast<int32_t>(tile_rows), keys);
    return tile_order_from_keys(
        dag, scratch, keys,
        static_cast<uint64_t>((n + tile_rows - 1) / tile_rows), stream);
}

extern "C" int lcdhip_dag_box_order(lcdhip_dag *dag, const int64_t grid[3],
                                    const int64_t box[3],
                                    lcdhip_stream stream_handle)
{
    LCDHIP_REQUIRE_INIT();
    if (!dag || !grid || !box) {
        set_error("dag/grid/box must not be NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    const int64_t n = dag->info.n;
    int64_t boxes[3];
    for (int axis = 0; axis < 3; ++axis) {
        if (grid[axis] <= 0 || box[axis] <= 0 || grid[axis] > 0x7fffffff ||
            box[axis] > 0x7fffffff) {
            set_error("grid and box extents must be positive 32-bit integers");
            return LCDHIP_ERR_ARGUMENT;
        }
        boxes[axis] = (grid[axis] + box[axis] - 1) / box[axis];
    }
    // (division, not the product: the product of three extents can overflow)
    if (n % grid[0] || (n / grid[0]) % grid[1] ||
        n / grid[0] / grid[1] != grid[2]) {
        set_error("a grid of %lld x %lld x %lld points does not have %lld nodes",
                  static_cast<long long>(grid[0]), static_cast<long long>(grid[1]),
                  static_cast<long long>(grid[2]), static_cast<long long>(n));
        return LCDHIP_ERR_ARGUMENT;
    }
    int status;
    if ((status = tile_order_ready(dag))) return status;
    hipStream_t stream = resolve_stream(stream_handle);
    if (n == 0) {
        if ((status = dag_alloc(dag, LCDHIP_DAG_TILE_NODES, 0))) return status;
        return dag_alloc(dag, LCDHIP_DAG_TILE_POS, 0);
    }
    Scratch scratch;
    uint32_t *keys = nullptr;
    LCDHIP_CHECK(scratch.alloc(&keys, n));
    hipLaunchKernelGGL(box_keys_kernel, dim3(blocks_for(n)), dim3(kBlock), 0,
                       stream, dag->arrays[LCDHIP_DAG_WAVEFRONTS], n,
                       static_cast<int32_t>(grid[0]), static_cast<int32_t>(grid[1]),
                       static_cast<int32_t>(box[0]), static_cast<int32_t>(box[1]),
                       static_cast<int32_t>(box[2]),
                       static_cast<int32_t>(boxes[0]), static_cast<int32_t>(boxes[1]),
                       keys);
    // n nodes make at most n boxes
    return tile_order_from_keys(
        dag, scratch, keys,
        static_cast<uint64_t>(boxes[0] * boxes[1] * boxes[2]), stream);
}

extern "C" int lcdhip_dag_edge_offsets(const lcdhip_dag *dag, int64_t capacity,
                                       int64_t *offsets_out, int64_t *counts_out,
                                       int64_t *distinct_out,
                                       lcdhip_stream stream_handle)
{
    LCDHIP_REQUIRE_INIT();
    if (!dag || capacity < 0 || !distinct_out ||
        (capacity > 0 && (!offsets_out || !counts_out))) {
        set_error("bad argument to lcdhip_dag_edge_offsets");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t stream = resolve_stream(stream_handle);
    const int64_t n = dag->info.n, edges = dag->info.edges;
    *distinct_out = 0;
    if (n == 0 || edges == 0)
        return LCDHIP_OK;
    if (edges > 0xffffffffll) {
        set_error("edge offsets of more than 2^32 edges");
        return LCDHIP_ERR_ARGUMENT;
    }
    Scratch scratch;
    uint32_t *offsets = nullptr, *sorted = nullptr, *unique = nullptr,
             *counts = nullptr, *runs = nullptr;
    LCDHIP_CHECK(scratch.alloc(&offsets, edges));
    LCDHIP_CHECK(scratch.alloc(&sorted, edges));
    LCDHIP_CHECK(scratch.alloc(&unique, edges));
    LCDHIP_CHECK(scratch.alloc(&counts, edges));
    LCDHIP_CHECK(scratch.alloc(&runs, 1));
    hipLaunchKernelGGL(edge_offsets_kernel, dim3(blocks_for(n)), dim3(kBlock), 0,
                       stream, dag->arrays[LCDHIP_DAG_PTR],
                       dag->arrays[LCDHIP_DAG_INDEX], n, offsets);
    size_t bytes = 0;
    char *temp = nullptr;
    LCDHIP_CHECK(rocprim::radix_sort_keys(nullptr, bytes, offsets, sorted,
                                          static_cast<size_t>(edges), 0, 32,
                                          stream));
    LCDHIP_CHECK(scratch.alloc(&temp, bytes));
    LCDHIP_CHECK(rocprim::radix_sort_keys(temp, bytes, offsets, sorted,
                                          static_cast<size_t>(edges), 0, 32,
                                          stream));
    size_t rle_bytes = 0;
    char *rle_temp = nullptr;
    LCDHIP_CHECK(rocprim::run_length_encode(
        nullptr, rle_bytes, sorted, static_cast<unsigned int>(edges), unique,
        counts, runs, stream));
    LCDHIP_CHECK(scratch.alloc(&rle_temp, rle_bytes));
    LCDHIP_CHECK(rocprim::run_length_encode(
        rle_temp, rle_bytes, sorted, static_cast<unsigned int>(edges), unique,
        counts, runs, stream));
    LCDHIP_CHECK(hipGetLastError());
    uint32_t distinct = 0;
    LCDHIP_CHECK(hipMemcpyAsync(&distinct, runs, 4, hipMemcpyDeviceToHost,
                                stream));
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    *distinct_out = distinct;
    const int64_t take = std::min<int64_t>(capacity, distinct);
    if (take > 0) {
        std::vector<uint32_t> host_unique(take), host_counts(take);
        LCDHIP_CHECK(hipMemcpy(host_unique.data(), unique, take * 4,
                               hipMemcpyDeviceToHost));
        LCDHIP_CHECK(hipMemcpy(host_counts.data(), counts, take * 4,
                               hipMemcpyDeviceToHost));
        for (int64_t k = 0; k < take; ++k) {
            offsets_out[k] = static_cast<int64_t>(host_unique[k]) - 0x80000000ll;
            counts_out[k] = host_counts[k];
        }
    }
    return LCDHIP_OK;
}

namespace {

__global__ void task_records_kernel(const int32_t *__restrict__ order,
                                    const int32_t *__restrict__ in_ptr,
                                    const int32_t *__restrict__ in_src,
                                    const int32_t *__restrict__ in_pos,
                                    const int32_t *__restrict__ position,
                                    int64_t n, int lanes,
                                    int32_t *__restrict__ rec_in,
                                    int32_t *__restrict__ rec_src,
                                    int32_t *__restrict__ rec_pos,
                                    unsigned long long *__restrict__ overflow)
{
    int64_t slot = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (slot >= n * lanes)
        return;
    const int64_t q = slot / lanes;
    const int lane = static_cast<int>(slot - q * lanes);
    const int32_t node = order[q];
    const int32_t begin = in_ptr[node], end = in_ptr[node + 1];
    if (lane == 0) {
        rec_in[2 * q] = begin;
        rec_in[2 * q + 1] = end;
        if (end - begin > lanes)
            atomicAdd(overflow, 1ull);
    }
    const bool has = begin + lane < end;
    int32_t source = has ? in_src[begin + lane] : 0;
    if (position) {
        // sources by their place in the task order; one that does not come
        // before its consumer would be waited for by a tile that runs first
        source = has ? position[source] : 0;
        if (has && source >= q)
            atomicAdd(overflow + 1, 1ull);
        if (lane == 0)
            for (int32_t e = begin + lanes; e < end; ++e)
                if (position[in_src[e]] >= q)
                    atomicAdd(overflow + 1, 1ull);
    }
    rec_src[slot] = source;
    rec_pos[slot] = has ? in_pos[begin + lane] : 0;
}

}

extern "C" int lcdhip_dag_task_records(lcdhip_dag *dag, int lanes, int tiled,
                                       lcdhip_stream stream_handle,
                                       int64_t *overflow_tasks_out)
{
    LCDHIP_REQUIRE_INIT();
    if (!dag || lanes < 1 || lanes > 64 || tiled < LCDHIP_RECORDS_LEVEL_ORDER ||
        tiled > LCDHIP_RECORDS_TILE_POSITIONS) {
        set_error("task records need a dag, 1 to 64 lanes per task and one of "
                  "the LCDHIP_RECORDS_* orders");
        return LCDHIP_ERR_ARGUMENT;
    }
    const int32_t *order = dag->arrays[tiled ? LCDHIP_DAG_TILE_NODES
                                             : LCDHIP_DAG_WAVEFRONTS];
    const int32_t *position = tiled == LCDHIP_RECORDS_TILE_POSITIONS
                                  ? dag->arrays[LCDHIP_DAG_TILE_POS] : nullptr;
    if (!order || dag->info.scheduled != dag->info.n ||
        !dag->arrays[LCDHIP_DAG_IN_PTR] ||
        (tiled == LCDHIP_RECORDS_TILE_POSITIONS && !position)) {
        set_error("task records need level sets that cover every node, the "
                  "incoming listing and, when tiled, the tile order");
        return LCDHIP_ERR_ARGUMENT;
    }
    hipStream_t stream = resolve_stream(stream_handle);
    const int64_t n = dag->info.n;
    if (n * lanes >= (int64_t(1) << 31)) {
        set_error("task records of %lld tasks x %d lanes exceed 2^31 entries",
                  static_cast<long long>(n), lanes);
        return LCDHIP_ERR_ARGUMENT;
    }
    for (int which : {LCDHIP_DAG_REC_IN, LCDHIP_DAG_REC_SRC, LCDHIP_DAG_REC_POS})
        dag_release(dag, which);
    int status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_REC_IN, 2 * n))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_REC_SRC, n * lanes))) return status;
    if ((status = dag_alloc(dag, LCDHIP_DAG_REC_POS, n * lanes))) return status;
    if (overflow_tasks_out)
        *overflow_tasks_out = 0;
    if (n == 0)
        return LCDHIP_OK;
    Scratch scratch;
    unsigned long long *d_overflow = nullptr;
    LCDHIP_CHECK(scratch.alloc(&d_overflow, 2));
    LCDHIP_CHECK(hipMemsetAsync(d_overflow, 0, 16, stream));
    hipLaunchKernelGGL(task_records_kernel, dim3(blocks_for(n * lanes)),
                       dim3(kBlock), 0, stream, order,
                       dag->arrays[LCDHIP_DAG_IN_PTR],
                       dag->arrays[LCDHIP_DAG_IN_SRC],
                       dag->arrays[LCDHIP_DAG_IN_POS], position, n, lanes,
                       dag->arrays[LCDHIP_DAG_REC_IN],
                       dag->arrays[LCDHIP_DAG_REC_SRC],
                       dag->arrays[LCDHIP_DAG_REC_POS], d_overflow);
    LCDHIP_CHECK(hipGetLastError());
    unsigned long long overflow[2] = {0, 0};
    LCDHIP_CHECK(hipMemcpyAsync(overflow, d_overflow, 16, hipMemcpyDeviceToHost,
                                stream));
    LCDHIP_CHECK(hipStreamSynchronize(stream));
    if (overflow[1]) {
        for (int which : {LCDHIP_DAG_REC_IN, LCDHIP_DAG_REC_SRC, LCDHIP_DAG_REC_POS})
            dag_release(dag, which);
        set_error("the tile order is not a topological order: %llu edges come "
                  "from a later position",
                  static_cast<unsigned long long>(overflow[1]));
        return LCDHIP_ERR_ARGUMENT;
    }
    if (overflow_tasks_out)
        *overflow_tasks_out = static_cast<int64_t>(overflow[0]);
    return LCDHIP_OK;
}

extern "C" int lcdhip_dag_get_info(const lcdhip_dag *dag, lcdhip_dag_info *out)
{
    if (!dag || !out) {
        set_error("dag/out must not be NULL");
        return LCDHIP_ERR_ARGUMENT;
    }
    *out = dag->info;
    return LCDHIP_OK;
}

extern "C" int lcdhip_dag_array(const lcdhip_dag *dag, int which, void **d_out,
                                int64_t *count_out)
{
    if (!dag || which < 0 || which >= LCDHIP_DAG_ARRAYS || !d_out || !count_out) {
        set_error("bad argument to lcdhip_dag_array");
        return LCDHIP_ERR_ARGUMENT;
    }
    if (!dag->arrays[which]) {
        set_error("DAG array %d was not built (levels not requested?)", which);
        return LCDHIP_ERR_ARGUMENT;
    }
    *d_out = dag->arrays[which];
    *count_out = dag->counts[which];
    return LCDHIP_OK;
}

extern "C" int lcdhip_dag_download(const lcdhip_dag *dag, int which,
                                   int32_t *host_out, int64_t capacity)
{
    LCDHIP_REQUIRE_INIT();
    void *d_ptr = nullptr;
    int64_t count = 0;
    int status = lcdhip_dag_array(dag, which, &d_ptr, &count);
    if (status)
        return status;
    if (capacity < count || (count > 0 && !host_out)) {
        set_error("host buffer too small: %lld < %lld",
                  static_cast<long long>(capacity), static_cast<long long>(count));
        return LCDHIP_ERR_ARGUMENT;
    }
    if (count > 0)
        LCDHIP_CHECK(hipMemcpy(host_out, d_ptr, count * 4, hipMemcpyDeviceToHost));
    return LCDHIP_OK;
}

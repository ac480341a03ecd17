/*
 * lcd_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * Single-threaded CPU restatement of the algorithms on the `@parallel`
 * execution path of SwiftWare-Lab/lcd.  It exists only so that tests, the
 * smoke check and the benchmark's CPU-baseline leg have something to compare
 * the HIP path against.  Nothing in the shipped package may link or load it.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off: no FMA contraction,
 * so the floating-point results are those of the Python loops).
 *
 * What each function restates (paths under the reference checkout):
 *   oracle_sptrsv_csc        README.md:85-92 (sptrsv_csc), demo/sptrsv.py:36-43
 *   oracle_sptrsv_csr        compiler/demo/sptrsv.py:26-33
 *   oracle_gauss_seidel_csr  compiler/demo/gauss_seidel.py:18-26
 *   oracle_ilu0_csr          compiler/demo/spilu0.py:21-47
 *   oracle_ilu0_csc          compiler/demo/spilu0.py:50-82
 *   oracle_dag_*             generated inspector, compiler/dag_codegen.py:1151-1550
 *                            (set successors, unique in-degree, edge
 *                            multiplicity), compact_successors
 *                            compiler/dag_preprocessing.py:115-143
 *   oracle_dag_levels        wavefronts_from_dag / preprocess_wavefront,
 *                            compiler/dag_preprocessing.py:146-204
 *   oracle_band_chains       _band_chains, compiler/dag_preprocessing.py:258-298
 *   oracle_lookup_positions  _materialize_lookup,
 *                            compiler/structural_lookups.py:279-333
 *
 * How it is pinned (tests/test_oracle_pins.py): the reference's own
 * known-answer vectors (tests/golden/reference_vectors.json), SciPy's
 * triangular solve, dense LU on dense patterns, closed-form stencil levels,
 * and a literal set-based pure-Python restatement on small random inputs.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ solvers */

void oracle_sptrsv_csc(const int32_t *Ap, const int32_t *Ai, const double *Ax,
                       const double *b, int64_t n, double *x)
{
    memset(x, 0, (size_t)n * sizeof(double));
    for (int64_t i = 0; i < n; ++i) {
        x[i] = (b[i] - x[i]) / Ax[Ap[i]];
        for (int64_t j = (int64_t)Ap[i] + 1; j < Ap[i + 1]; ++j)
            x[Ai[j]] += Ax[j] * x[i];
    }
}

void oracle_sptrsv_csr(const int32_t *Ap, const int32_t *Ai, const double *Ax,
                       const double *b, int64_t n, double *x)
{
    memset(x, 0, (size_t)n * sizeof(double));
    for (int64_t i = 0; i < n; ++i) {
        x[i] = b[i];
        for (int64_t j = Ap[i]; j < (int64_t)Ap[i + 1] - 1; ++j)
            x[i] -= Ax[j] * x[Ai[j]];
        x[i] /= Ax[Ap[i + 1] - 1];
    }
}

void oracle_gauss_seidel_csr(const int32_t *Ap, const int32_t *Ai,
                             const double *Ax, const double *D, const double *b,
                             double *x, int64_t n, int64_t max_iter)
{
    for (int64_t sweep = 0; sweep < max_iter; ++sweep)
        for (int64_t i = 0; i < n; ++i) {
            x[i] = b[i];
            for (int64_t j = Ap[i]; j < Ap[i + 1]; ++j)
                x[i] -= Ax[j] * x[Ai[j]];
            x[i] /= D[i];
        }
}

void oracle_ilu0_csr(double *A_data, const int32_t *A_indices,
                     const int32_t *A_indptr, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) {
        int64_t row_start = A_indptr[i], row_end = A_indptr[i + 1];
        for (int64_t k_ptr = row_start; k_ptr < row_end; ++k_ptr) {
            int64_t k = A_indices[k_ptr];
            if (k >= i)
                break;
            double diag_val = 0.0;
            for (int64_t d = A_indptr[k]; d < A_indptr[k + 1]; ++d)
                if (A_indices[d] == k) {
                    diag_val = A_data[d];
                    break;
                }
            if (diag_val != 0.0) {
                A_data[k_ptr] = A_data[k_ptr] / diag_val;
                double l_ik = A_data[k_ptr];
                for (int64_t j_ptr = k_ptr + 1; j_ptr < row_end; ++j_ptr) {
                    int64_t j = A_indices[j_ptr];
                    for (int64_t kj = A_indptr[k]; kj < A_indptr[k + 1]; ++kj)
                        if (A_indices[kj] == j) {
                            double u_kj = A_data[kj];
                            A_data[j_ptr] = A_data[j_ptr] - l_ik * u_kj;
                            break;
                        }
                }
            }
        }
    }
}

/* Right-looking ILU0 on CSC storage: column k scales its sub-diagonal and
 * updates every later column j that holds an entry in row k. */
void oracle_ilu0_csc(double *A_data, const int32_t *A_indices,
                     const int32_t *A_indptr, int64_t n)
{
    for (int64_t k = 0; k < n; ++k) {
        int64_t col_start = A_indptr[k], col_end = A_indptr[k + 1];
        double diag_val = 0.0;
        for (int64_t d = col_start; d < col_end; ++d)
            if (A_indices[d] == k) {
                diag_val = A_data[d];
                break;
            }
        for (int64_t i_ptr = col_start; i_ptr < col_end; ++i_ptr) {
            int64_t i = A_indices[i_ptr];
            if (i <= k)
                continue;
            if (diag_val != 0.0) {
                A_data[i_ptr] = A_data[i_ptr] / diag_val;
                double l_ik = A_data[i_ptr];
                for (int64_t j = k + 1; j < n; ++j) {
                    int64_t j_start = A_indptr[j], j_end = A_indptr[j + 1];
                    double u_kj = 0.0;
                    for (int64_t kj = j_start; kj < j_end; ++kj)
                        if (A_indices[kj] == k) {
                            u_kj = A_data[kj];
                            break;
                        }
                    if (u_kj != 0.0)
                        for (int64_t ij = j_start; ij < j_end; ++ij)
                            if (A_indices[ij] == i) {
                                A_data[ij] = A_data[ij] - l_ik * u_kj;
                                break;
                            }
                }
            }
        }
    }
}

/* True flop count of ILU0-CSR: one division per eliminated entry plus a
 * multiply-subtract per matched (j, k) pair. */
int64_t oracle_ilu0_csr_flops(const int32_t *A_indices, const int32_t *A_indptr,
                              int64_t n)
{
    int64_t flops = 0;
    for (int64_t i = 0; i < n; ++i) {
        int64_t row_end = A_indptr[i + 1];
        for (int64_t k_ptr = A_indptr[i]; k_ptr < row_end; ++k_ptr) {
            int64_t k = A_indices[k_ptr];
            if (k >= i)
                break;
            flops += 1;
            for (int64_t j_ptr = k_ptr + 1; j_ptr < row_end; ++j_ptr) {
                int64_t j = A_indices[j_ptr];
                for (int64_t kj = A_indptr[k]; kj < A_indptr[k + 1]; ++kj)
                    if (A_indices[kj] == j) {
                        flops += 2;
                        break;
                    }
            }
        }
    }
    return flops;
}

/* --------------------------------------------------------------------- DAG */

/* One edge rule of the generated inspector, restricted to the shape every
 * supported loop produces: an outer loop over the n tasks and an inner loop
 * over a pointer-delimited segment.
 *
 *   for seg in range(n):
 *       for p in range(ptr[seg] + lower_offset, ptr[seg + 1] + upper_offset):
 *           if break_at_owner and idx[p] >= seg: break
 *           (src, dst) = (seg, idx[p]) if owner_is_source else (idx[p], seg)
 *           if guard(src, dst): successors[src].add(dst); edge_count[dst] += 1
 *
 * guard: 0 = none, 1 = dst > src, 2 = src != dst.
 *
 * relation 1 (no arrays): `for j in range(seg + lower_offset, n)` yields
 * seg -> j, the planner's output for a relational loop
 * (compiler/transform_tests/test_spilu0_codegen.py:146-150).
 */
typedef struct {
    const int32_t *ptr;
    const int32_t *idx;
    int32_t owner_is_source;
    int32_t lower_offset;
    int32_t upper_offset;
    int32_t guard;
    int32_t break_at_owner;
    int32_t relation;
} oracle_rule;

typedef struct {
    int64_t n;
    int64_t edges;          /* unique edges */
    int64_t levels;
    int64_t scheduled;      /* nodes covered by the level sets (< n: cycle) */
    int32_t *dag_ptr;       /* n + 1 */
    int32_t *dag_index;     /* edges, sorted and unique per source */
    int32_t *dep_count;     /* unique in-degree */
    int32_t *edge_count;    /* multiplicity of rule hits per destination */
    int32_t *level_of;      /* -1 when unscheduled */
    int32_t *wavefronts;    /* scheduled nodes by (level, id) */
    int32_t *wavefront_ptr; /* levels + 1 */
    int32_t status;         /* 0 ok, 1 endpoint out of range */
} oracle_dag;

static int cmp_i32(const void *a, const void *b)
{
    int32_t x = *(const int32_t *)a, y = *(const int32_t *)b;
    return (x > y) - (x < y);
}

typedef void (*edge_fn)(void *state, int64_t src, int64_t dst);

static int enumerate_rule(const oracle_rule *r, int64_t n, edge_fn fn, void *st)
{
    if (r->relation == 1) {
        for (int64_t seg = 0; seg < n; ++seg)
            for (int64_t j = seg + r->lower_offset; j < n; ++j)
                fn(st, seg, j);
        return 0;
    }
    if (r->relation == 2) {
        /* chain rule: seg -> seg + lower_offset */
        for (int64_t seg = 0; seg + r->lower_offset < n; ++seg)
            fn(st, seg, seg + r->lower_offset);
        return 0;
    }
    for (int64_t seg = 0; seg < n; ++seg) {
        int64_t lo = (int64_t)r->ptr[seg] + r->lower_offset;
        int64_t hi = (int64_t)r->ptr[seg + 1] + r->upper_offset;
        for (int64_t p = lo; p < hi; ++p) {
            int64_t other = r->idx[p];
            if (r->break_at_owner && other >= seg)
                break;
            int64_t src = r->owner_is_source ? seg : other;
            int64_t dst = r->owner_is_source ? other : seg;
            if (r->guard == 1 && !(dst > src))
                continue;
            if (r->guard == 2 && src == dst)
                continue;
            if (other < 0 || other >= n)
                return 1;
            fn(st, src, dst);
        }
    }
    return 0;
}

typedef struct {
    int64_t *count;
    int32_t *edge_count;
    int32_t *fill;
    int64_t *cursor;
} edge_state;

static void count_edge(void *s, int64_t src, int64_t dst)
{
    edge_state *st = (edge_state *)s;
    st->count[src] += 1;
    st->edge_count[dst] += 1;
}

static void fill_edge(void *s, int64_t src, int64_t dst)
{
    edge_state *st = (edge_state *)s;
    st->fill[st->cursor[src]++] = (int32_t)dst;
}

void oracle_dag_free(oracle_dag *d)
{
    if (!d)
        return;
    free(d->dag_ptr); free(d->dag_index); free(d->dep_count);
    free(d->edge_count); free(d->level_of); free(d->wavefronts);
    free(d->wavefront_ptr); free(d);
}

/* Levels by the reference's Kahn iteration: the first wavefront is every
 * node with in-degree 0 in ascending id; each next wavefront is the sorted
 * set of nodes whose remaining count reaches 0 while the current one is
 * released. */
static void kahn_levels(oracle_dag *d)
{
    int64_t n = d->n;
    int32_t *remaining = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    memcpy(remaining, d->dep_count, (size_t)n * 4);
    d->level_of = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    d->wavefronts = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    int64_t cap = 16, levels = 0;
    int32_t *wptr = (int32_t *)malloc((size_t)cap * 4);
    wptr[0] = 0;
    for (int64_t v = 0; v < n; ++v)
        d->level_of[v] = -1;
    int64_t begin = 0, end = 0;
    for (int64_t v = 0; v < n; ++v)
        if (remaining[v] == 0)
            d->wavefronts[end++] = (int32_t)v;
    while (end > begin) {
        if (levels + 2 > cap) {
            cap *= 2;
            wptr = (int32_t *)realloc(wptr, (size_t)cap * 4);
        }
        int64_t next_end = end;
        for (int64_t q = begin; q < end; ++q) {
            int32_t v = d->wavefronts[q];
            d->level_of[v] = (int32_t)levels;
            for (int64_t e = d->dag_ptr[v]; e < d->dag_ptr[v + 1]; ++e) {
                int32_t w = d->dag_index[e];
                if (--remaining[w] == 0)
                    d->wavefronts[next_end++] = w;
            }
        }
        qsort(d->wavefronts + end, (size_t)(next_end - end), 4, cmp_i32);
        levels += 1;
        wptr[levels] = (int32_t)end;
        begin = end;
        end = next_end;
    }
    d->levels = levels;
    d->scheduled = end;
    d->wavefront_ptr = wptr;
    free(remaining);
}

oracle_dag *oracle_dag_build(const oracle_rule *rules, int32_t rule_count,
                             int64_t n)
{
    oracle_dag *d = (oracle_dag *)calloc(1, sizeof(oracle_dag));
    d->n = n;
    size_t nn = (size_t)(n ? n : 1);
    int64_t *count = (int64_t *)calloc(nn + 1, sizeof(int64_t));
    d->edge_count = (int32_t *)calloc(nn, 4);
    d->dep_count = (int32_t *)calloc(nn, 4);
    d->dag_ptr = (int32_t *)calloc(nn + 1, 4);
    edge_state st = {count, d->edge_count, NULL, NULL};
    for (int32_t r = 0; r < rule_count; ++r)
        if (enumerate_rule(&rules[r], n, count_edge, &st)) {
            d->status = 1;
            free(count);
            return d;
        }
    int64_t *cursor = (int64_t *)malloc((nn + 1) * sizeof(int64_t));
    int64_t total = 0;
    for (int64_t v = 0; v < n; ++v) {
        cursor[v] = total;
        total += count[v];
    }
    cursor[n] = total;
    int32_t *raw = (int32_t *)malloc((size_t)(total ? total : 1) * 4);
    int64_t *start = (int64_t *)malloc((nn + 1) * sizeof(int64_t));
    memcpy(start, cursor, (nn + 1) * sizeof(int64_t));
    st.fill = raw;
    st.cursor = cursor;
    for (int32_t r = 0; r < rule_count; ++r)
        enumerate_rule(&rules[r], n, fill_edge, &st);
    /* set semantics: sort and deduplicate each successor list in place */
    int64_t unique = 0;
    for (int64_t v = 0; v < n; ++v) {
        int64_t lo = start[v], hi = start[v] + count[v];
        qsort(raw + lo, (size_t)(hi - lo), 4, cmp_i32);
        d->dag_ptr[v] = (int32_t)unique;
        for (int64_t e = lo; e < hi; ++e)
            if (e == lo || raw[e] != raw[e - 1]) {
                raw[unique++] = raw[e];
                d->dep_count[raw[unique - 1]] += 1;
            }
    }
    d->dag_ptr[n] = (int32_t)unique;
    d->edges = unique;
    d->dag_index = raw;
    free(count); free(cursor); free(start);
    kahn_levels(d);
    return d;
}

/* Same data structure from explicit successor lists (for DAGs that do not
 * come from a segment rule, e.g. the cyclic known-answer case). */
oracle_dag *oracle_dag_from_successors(const int32_t *succ_ptr,
                                       const int32_t *succ_index, int64_t n)
{
    oracle_dag *d = (oracle_dag *)calloc(1, sizeof(oracle_dag));
    d->n = n;
    size_t nn = (size_t)(n ? n : 1);
    int64_t total = succ_ptr[n];
    d->edge_count = (int32_t *)calloc(nn, 4);
    d->dep_count = (int32_t *)calloc(nn, 4);
    d->dag_ptr = (int32_t *)calloc(nn + 1, 4);
    int32_t *raw = (int32_t *)malloc((size_t)(total ? total : 1) * 4);
    memcpy(raw, succ_index, (size_t)total * 4);
    int64_t unique = 0;
    for (int64_t v = 0; v < n; ++v) {
        int64_t lo = succ_ptr[v], hi = succ_ptr[v + 1];
        for (int64_t e = lo; e < hi; ++e) {
            if (raw[e] < 0 || raw[e] >= n) {
                d->status = 1;
                d->dag_index = raw;
                return d;
            }
            d->edge_count[raw[e]] += 1;
        }
        qsort(raw + lo, (size_t)(hi - lo), 4, cmp_i32);
        d->dag_ptr[v] = (int32_t)unique;
        for (int64_t e = lo; e < hi; ++e)
            if (e == lo || raw[e] != raw[e - 1]) {
                raw[unique++] = raw[e];
                d->dep_count[raw[unique - 1]] += 1;
            }
    }
    d->dag_ptr[n] = (int32_t)unique;
    d->edges = unique;
    d->dag_index = raw;
    kahn_levels(d);
    return d;
}

/* Chains of connected nodes inside bands of `band_width` consecutive levels.
 * Components are listed in order of their first member in band order; members
 * keep band order.  Outputs: task_nodes[n], task_ptr[<= n + 1],
 * band_ptr[ceil(levels / band_width) + 1]; returns the task count. */
int64_t oracle_band_chains(const oracle_dag *d, int64_t band_width,
                           int32_t *task_nodes, int32_t *task_ptr,
                           int32_t *band_ptr)
{
    int64_t n = d->n, tasks = 0, out = 0, bands = 0;
    int32_t *local = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    int32_t *parent = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    int32_t *chain_of = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    int32_t *chain_size = (int32_t *)malloc((size_t)(n ? n : 1) * 4);
    for (int64_t v = 0; v < n; ++v)
        local[v] = -1;
    task_ptr[0] = 0;
    band_ptr[0] = 0;
    for (int64_t first = 0; first < d->levels; first += band_width) {
        int64_t last = first + band_width < d->levels ? first + band_width
                                                       : d->levels;
        const int32_t *band = d->wavefronts + d->wavefront_ptr[first];
        int64_t size = d->wavefront_ptr[last] - d->wavefront_ptr[first];
        for (int64_t p = 0; p < size; ++p) {
            local[band[p]] = (int32_t)p;
            parent[p] = (int32_t)p;
        }
        for (int64_t p = 0; p < size; ++p) {
            int32_t v = band[p];
            for (int64_t e = d->dag_ptr[v]; e < d->dag_ptr[v + 1]; ++e) {
                int32_t q = local[d->dag_index[e]];
                if (q < 0)
                    continue;
                int32_t a = (int32_t)p, b = q;
                while (parent[a] != a) { parent[a] = parent[parent[a]]; a = parent[a]; }
                while (parent[b] != b) { parent[b] = parent[parent[b]]; b = parent[b]; }
                if (a != b)
                    parent[b] = a;
            }
        }
        /* number the components by first appearance, then bucket */
        int64_t comps = 0;
        for (int64_t p = 0; p < size; ++p) chain_of[p] = -1;
        int32_t *root_id = chain_of; /* indexed by root position */
        int32_t *member = (int32_t *)malloc((size_t)(size > 0 ? size : 1) * 4);
        for (int64_t p = 0; p < size; ++p) {
            int32_t r = (int32_t)p;
            while (parent[r] != r) r = parent[r];
            if (root_id[r] < 0) {
                root_id[r] = (int32_t)comps;
                chain_size[comps++] = 0;
            }
            member[p] = root_id[r];
            chain_size[member[p]] += 1;
        }
        int64_t base = out;
        for (int64_t c = 0; c < comps; ++c) {
            int32_t sz = chain_size[c];
            chain_size[c] = (int32_t)base; /* becomes the write cursor */
            base += sz;
            task_ptr[tasks + c + 1] = (int32_t)base;
        }
        for (int64_t p = 0; p < size; ++p)
            task_nodes[chain_size[member[p]]++] = band[p];
        out = base;
        tasks += comps;
        band_ptr[++bands] = (int32_t)tasks;
        for (int64_t p = 0; p < size; ++p)
            local[band[p]] = -1;
        free(member);
    }
    free(local); free(parent); free(chain_of); free(chain_size);
    return tasks;
}

/* Position of the entry idx[p] == segment inside every segment, or -1.
 * Returns 0, or 1 for a non-monotone / out-of-range pointer array, or 2 for
 * an unsorted segment (both are StructuralLookupError in the reference). */
int32_t oracle_lookup_positions(const int32_t *ptr, const int32_t *idx,
                                int64_t n, int64_t idx_size, int32_t *positions)
{
    int64_t previous = ptr[0];
    if (previous < 0 || previous > idx_size)
        return 1;
    for (int64_t s = 0; s < n; ++s) {
        int64_t start = ptr[s], end = ptr[s + 1];
        positions[s] = -1;
        if (start < previous || end < start || end > idx_size)
            return 1;
        for (int64_t p = start + 1; p < end; ++p)
            if (idx[p] < idx[p - 1])
                return 2;
        /* first position with idx[p] >= s (searchsorted side="left") */
        int64_t lo = start, hi = end;
        while (lo < hi) {
            int64_t mid = (lo + hi) / 2;
            if (idx[mid] < s) lo = mid + 1; else hi = mid;
        }
        if (lo < end && idx[lo] == s)
            positions[s] = (int32_t)lo;
        previous = end;
    }
    return 0;
}

"""Time the generated solvers over a list of Matrix Market files.

Counterpart of the reference's benchmark drivers (benchmark/bench_utils.py:
64-80 reads a list of file names below a base directory and orders it by
entry count; benchmark/sptrsv_benchmark.py:626-630 and
benchmark/spilu0_benchmark.py:767 report the median of repeated launches as
``(n + 2 nnz) / t`` and ``2 nnz / t``).  Each matrix goes through the
reference's regulariser (compiler/demo/matrix.py:45-81), its lower triangle is
solved in CSC and CSR form and the whole matrix is factorised by CSR ILU0,
with the schedule the decorator's scheduler picks unless options fix it.

    python -m lcd_amd.demo.matrix_bench matrix_list.txt /data/suitesparse/

prints one CSV line per (matrix, kernel).
"""

import os
import sys

import numpy as np

from lcd_amd import hip_runtime
from lcd_amd.demo import spilu0, sptrsv
from lcd_amd.demo.matrix import (load_matrix_market, lower_triangle,
                                 manufactured_rhs)

KERNELS = ("sptrsv_csc", "sptrsv_csr", "ilu0_csr")
COLUMNS = ("matrix", "kernel", "n", "nnz", "levels", "execution_mode",
           "dependence_protocol", "threads_per_block", "task_lanes",
           "median_ms", "p20_ms", "p80_ms", "gflops", "max_abs_error",
           "inspect_compile_ms")


def matrix_list(list_path, base_path=""):
    """Paths named in ``list_path`` (one per line, below ``base_path``), in
    ascending order of the entry count their headers declare."""
    with open(list_path) as handle:
        names = [line.strip() for line in handle if line.strip()]
    paths = [os.path.join(base_path, name) for name in names]

    def declared_entries(path):
        with open(path, "rb") as handle:
            for raw in handle:
                line = raw.decode("ascii", "replace").strip()
                if line and not line.startswith("%"):
                    return int(line.split()[-1])
        return 0

    return [path for _, path in sorted(
        (declared_entries(path), path) for path in paths)]


def do_bench(step, device, warmup=5, repeats=20, quantiles=(0.5, 0.2, 0.8)):
    """Quantiles (ms) of ``repeats`` event-timed calls of ``step`` after
    ``warmup`` untimed ones."""
    for _ in range(warmup):
        step()
    device.synchronize()
    times = []
    start, stop = device.event(), device.event()
    for _ in range(repeats):
        device.record(start)
        step()
        device.record(stop)
        device.synchronize()
        times.append(device.elapsed_ms(start, stop))
    return [float(np.quantile(times, q)) for q in quantiles]


def bench_kernel(kernel, matrix, device, warmup=5, repeats=20, **options):
    """One result row (a dict over ``COLUMNS`` without ``matrix``)."""
    import time
    started = time.perf_counter()
    if kernel == "ilu0_csr":
        indptr = matrix.indptr.astype(np.int32)
        indices = matrix.indices.astype(np.int32)
        data = np.ascontiguousarray(matrix.data, dtype=np.float64)
        solver = spilu0.compile_ilu0_csr(
            execution_mode=options.pop("execution_mode", None),
            threads_per_block=options.pop("threads_per_block", None),
            **options)
        pristine = device.to_device(data)
        operands = [device.to_device(data), device.to_device(indices),
                    device.to_device(indptr)]
        call = solver.bind(*operands)
        flops = 2.0 * len(data)

        def step():
            device.copy(operands[0], pristine)      # factorised in place
            call.launch()
    else:
        storage = kernel[-3:]
        indptr, indices, data = lower_triangle(matrix, storage)
        rhs, expected = manufactured_rhs(indptr, indices, data, storage)
        compile_solver = (sptrsv.compile_sptrsv_csc if storage == "csc"
                          else sptrsv.compile_sptrsv_csr)
        solver = compile_solver(**options)
        operands = [device.to_device(a) for a in (indptr, indices, data, rhs)]
        call = solver.bind(*operands, len(rhs))
        flops = len(rhs) + 2.0 * len(data)
        step = call.launch
    device.synchronize()
    setup_ms = (time.perf_counter() - started) * 1e3
    step()
    call.synchronize()
    result = np.asarray(call.result())
    if kernel == "ilu0_csr":
        error = _ilu0_pattern_error(matrix, result)
    else:
        error = float(np.max(np.abs(result - expected)))
    median, low, high = do_bench(step, device, warmup, repeats)
    schedule = solver.current_schedule
    plan = solver.schedule_plan(*operands, *(
        [] if kernel == "ilu0_csr" else [len(rhs)]))
    return {
        "kernel": kernel, "n": matrix.shape[0], "nnz": len(data),
        "levels": plan.dag.levels,
        "execution_mode": schedule.execution_mode,
        "dependence_protocol": solver.hip_lowering.dependence_protocol,
        "threads_per_block": schedule.threads_per_block,
        "task_lanes": solver.hip_lowering.task_lanes,
        "median_ms": median, "p20_ms": low, "p80_ms": high,
        "gflops": flops / (median * 1e-3) / 1e9, "max_abs_error": error,
        "inspect_compile_ms": setup_ms,
    }


def _ilu0_pattern_error(matrix, factor):
    """max |(L U - A)| over the pattern: zero for an exact ILU0."""
    from scipy.sparse import csr_matrix, identity, tril, triu
    lu = csr_matrix((factor, matrix.indices, matrix.indptr),
                    shape=matrix.shape)
    product = (tril(lu, -1) + identity(matrix.shape[0])) @ triu(lu)
    pattern = csr_matrix((np.ones_like(matrix.data), matrix.indices,
                          matrix.indptr), shape=matrix.shape)
    difference = (product - matrix).multiply(pattern)
    return float(abs(difference).max()) if difference.nnz else 0.0


def run(list_path, base_path="", kernels=KERNELS, max_size=0, warmup=5,
        repeats=20, out=sys.stdout, **options):
    """Benchmark every listed matrix; returns the rows and prints them as
    CSV while it goes.  ``max_size`` > 0 keeps the leading principal block."""
    device = hip_runtime.default_device()
    print(",".join(COLUMNS), file=out, flush=True)
    rows = []
    for path in matrix_list(list_path, base_path):
        matrix = load_matrix_market(path, max_size).tocsr()
        matrix.sort_indices()
        for kernel in kernels:
            row = {"matrix": os.path.basename(path)}
            row.update(bench_kernel(kernel, matrix, device, warmup, repeats,
                                    **dict(options)))
            rows.append(row)
            print(",".join(
                f"{row[c]:.6g}" if isinstance(row[c], float) else str(row[c])
                for c in COLUMNS), file=out, flush=True)
    return rows


def main(argv=None):
    import argparse
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("list", help="text file with one .mtx name per line")
    parser.add_argument("base", nargs="?", default="",
                        help="directory the names are relative to")
    parser.add_argument("--kernels", default=",".join(KERNELS))
    parser.add_argument("--max-n", type=int, default=0,
                        help="leading principal sample size; 0 = full matrix")
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--repeats", type=int, default=20)
    parser.add_argument("--execution-mode", default=None,
                        choices=("wavefront", "sync_free"))
    args = parser.parse_args(argv)
    kernels = tuple(k for k in args.kernels.split(",") if k)
    unknown = [k for k in kernels if k not in KERNELS]
    if unknown:
        parser.error(f"unknown kernels {unknown}; choose from {KERNELS}")
    options = {}
    if args.execution_mode:
        options["execution_mode"] = args.execution_mode
    run(args.list, args.base, kernels, args.max_n, args.warmup, args.repeats,
        **options)


if __name__ == "__main__":
    main()

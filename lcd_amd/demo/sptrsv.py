"""CSR and CSC sparse triangular solves through ``@parallel``.

The loop bodies are the user loops of the reference (README.md:85-92,
compiler/demo/sptrsv.py:26-43); only the import changes.
"""

import numpy as np

from lcd_amd import parallel

FUNCTION_PROPS_CSR = {
    "Ap": ["monotonically_increasing"],
    "Ai": [],
}

FUNCTION_PROPS_CSC = {
    "Ap": ["monotonically_increasing"],
    "Ai": [],
    ("Ap", "Ai"): ["triangularity"],
}


def sptrsv_csc_loop(Ap, Ai, Ax, b, n):
    x = np.zeros(n)
    for i in range(n):
        x[i] = (b[i] - x[i]) / Ax[Ap[i]]
        for j in range(Ap[i] + 1, Ap[i + 1]):
            x[Ai[j]] += Ax[j] * x[i]
    return x


def sptrsv_csr_loop(Ap, Ai, Ax, b, n):
    x = np.zeros(n)
    for i in range(n):
        x[i] = b[i]
        for j in range(Ap[i], Ap[i + 1] - 1):
            x[i] -= Ax[j] * x[Ai[j]]
        x[i] /= Ax[Ap[i + 1] - 1]
    return x


def compile_sptrsv_csc(**options):
    """README form: ``block_map="i", thread_map="j"`` plus any overrides."""
    settings = dict(block_map="i", thread_map="j",
                    function_props=FUNCTION_PROPS_CSC)
    settings.update(options)
    return parallel(**settings)(sptrsv_csc_loop)


def compile_sptrsv_csr(**options):
    settings = dict(block_map="i", thread_map="j",
                    function_props=FUNCTION_PROPS_CSR)
    settings.update(options)
    return parallel(**settings)(sptrsv_csr_loop)


@parallel(loop="i", function_props=FUNCTION_PROPS_CSR, execution_mode="wavefront", threads_per_block=128)
def simple_sptrsv_csr(Ap, Ai, Ax, b, n):
    x = np.zeros(n)
    for i in range(n):
        x[i] = b[i]
        for j in range(Ap[i], Ap[i + 1] - 1):
            x[i] -= Ax[j] * x[Ai[j]]
        x[i] /= Ax[Ap[i + 1] - 1]
    return x


@parallel(loop="i", function_props=FUNCTION_PROPS_CSC, execution_mode="wavefront", threads_per_block=128)
def simple_sptrsv_csc(Ap, Ai, Ax, b, n):
    x = np.zeros(n)
    for i in range(n):
        x[i] = (b[i] - x[i]) / Ax[Ap[i]]
        for j in range(Ap[i] + 1, Ap[i + 1]):
            x[Ai[j]] += Ax[j] * x[i]
    return x


def run_demo(matrix_path, max_size=None, storage="both", verbose=True,
             **options):
    """Solve ``L x = b`` for the lower triangle of a Matrix Market input with
    the generated CSR and/or CSC solver (compiler/demo/sptrsv.py:44-78);
    returns ``{storage: (x, max_abs_error)}`` against the manufactured
    solution ``linspace(1, 2, n)``."""
    from lcd_amd.demo.matrix import (DEFAULT_MAX_N, load_matrix_market,
                                     lower_triangle, manufactured_rhs)
    source = load_matrix_market(
        matrix_path, DEFAULT_MAX_N if max_size is None else max_size)
    compilers = {"csr": compile_sptrsv_csr, "csc": compile_sptrsv_csc}
    selected = compilers if storage == "both" else {storage: compilers[storage]}
    results = {}
    for name, compile_solver in selected.items():
        indptr, indices, data = lower_triangle(source, name)
        rhs, expected = manufactured_rhs(indptr, indices, data, name)
        solver = compile_solver(**options)
        result = solver(indptr, indices, data, rhs, len(rhs))
        error = float(np.max(np.abs(result - expected)))
        results[name] = (result, error)
        if verbose:
            print(f"SpTRSV {name.upper()}: n={len(rhs)}, nnz={len(data)}, "
                  f"max_abs_error={error:.3e}")
    return results


def main(argv=None):
    import argparse
    parser = argparse.ArgumentParser(
        description="Run generated CSR/CSC SpTRSV on a Matrix Market input.")
    parser.add_argument("matrix",
                        help="path to a square real Matrix Market file")
    parser.add_argument("--max-n", type=int, default=None,
                        help="leading principal sample size; 0 = full matrix")
    parser.add_argument("--storage", choices=("csr", "csc", "both"),
                        default="both")
    parser.add_argument("--execution-mode", default=None,
                        choices=("wavefront", "sync_free"))
    args = parser.parse_args(argv)
    if args.max_n is not None and args.max_n < 0:
        parser.error("--max-n must be nonnegative")
    options = {}
    if args.execution_mode:
        options["execution_mode"] = args.execution_mode
    run_demo(args.matrix, args.max_n, args.storage, **options)


if __name__ == "__main__":
    main()

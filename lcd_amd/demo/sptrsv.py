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

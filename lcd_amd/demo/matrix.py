"""Matrix Market input for the demos and the benchmark harness.

Counterpart of compiler/demo/matrix.py:26-81 of the reference: read a square
real matrix, optionally keep its leading principal block, and regularise it
(values scaled to max |a| = 1, diagonal replaced by 1 + the row's absolute
off-diagonal sum) so that triangular solves and ILU0 meet no zero pivot.  The
reader is self-contained (coordinate and array formats; real, integer and
pattern fields; general, symmetric and skew-symmetric storage) and returns
SciPy CSR matrices; triangles for the solvers come from ``lower_triangle``.
"""

import gzip
from pathlib import Path

import numpy as np
import scipy.sparse as sp

DEFAULT_MAX_N = 128


class MatrixMarketError(ValueError):
    """The file is not a Matrix Market matrix this reader handles."""


def _open(path):
    path = Path(path)
    if path.suffix == ".gz":
        return gzip.open(path, "rt")
    return open(path, "r")


def read_matrix_market(path):
    """Parse one ``.mtx`` (or ``.mtx.gz``) file into a SciPy CSR matrix.

    Duplicate coordinate entries are summed, as SciPy's reader does."""
    path = Path(path).expanduser()
    if not path.is_file():
        raise FileNotFoundError(f"Matrix Market input not found: {path}")
    with _open(path) as handle:
        banner = handle.readline().split()
        if (len(banner) != 5 or banner[0] != "%%MatrixMarket"
                or banner[1].lower() != "matrix"):
            raise MatrixMarketError(f"Not a Matrix Market matrix file: {path}")
        layout, field, symmetry = (word.lower() for word in banner[2:])
        if layout not in ("coordinate", "array"):
            raise MatrixMarketError(f"Unknown Matrix Market format {layout!r}.")
        if field == "complex":
            raise MatrixMarketError(
                "Complex Matrix Market inputs are not supported yet.")
        if field not in ("real", "double", "integer", "pattern"):
            raise MatrixMarketError(f"Unknown Matrix Market field {field!r}.")
        if symmetry not in ("general", "symmetric", "skew-symmetric"):
            raise MatrixMarketError(
                f"Unsupported Matrix Market symmetry {symmetry!r}.")
        line = handle.readline()
        while line and (line.startswith("%") or not line.strip()):
            line = handle.readline()
        sizes = line.split()
        body = np.loadtxt(handle, dtype=np.float64, comments="%", ndmin=2)
    if layout == "coordinate":
        if len(sizes) != 3:
            raise MatrixMarketError("Bad coordinate size line.")
        rows, cols, entries = (int(word) for word in sizes)
        width = 2 if field == "pattern" else 3
        if body.size == 0:
            body = np.zeros((0, width))
        if body.shape != (entries, width):
            raise MatrixMarketError(
                f"Expected {entries} entries of {width} fields, found an "
                f"array of shape {body.shape}.")
        row = body[:, 0].astype(np.int64) - 1
        col = body[:, 1].astype(np.int64) - 1
        if entries and (row.min() < 0 or col.min() < 0 or row.max() >= rows
                        or col.max() >= cols):
            raise MatrixMarketError("A coordinate lies outside the matrix.")
        data = np.ones(entries) if field == "pattern" else body[:, 2].copy()
        if symmetry != "general":
            off = row != col
            sign = -1.0 if symmetry == "skew-symmetric" else 1.0
            row, col, data = (np.concatenate((row, col[off])),
                              np.concatenate((col, row[off])),
                              np.concatenate((data, sign * data[off])))
        matrix = sp.coo_matrix((data, (row, col)), shape=(rows, cols)).tocsr()
    else:
        if len(sizes) != 2 or field == "pattern":
            raise MatrixMarketError("Bad array size line.")
        rows, cols = (int(word) for word in sizes)
        values = body.ravel()
        dense = np.zeros((rows, cols))
        if symmetry == "general":
            if values.size != rows * cols:
                raise MatrixMarketError("Array body has the wrong length.")
            dense = values.reshape((cols, rows)).T.copy()
        else:
            skew = symmetry == "skew-symmetric"
            position = 0
            for c in range(cols):
                first = c + 1 if skew else c
                count = rows - first
                dense[first:, c] = values[position:position + count]
                position += count
            if position != values.size:
                raise MatrixMarketError("Array body has the wrong length.")
            lower = np.tril(dense, -1)
            dense = dense + (-lower.T if skew else lower.T)
        matrix = sp.csr_matrix(dense)
    matrix.sum_duplicates()
    return matrix


def regularize(matrix):
    """Normalise the values and make the diagonal strictly dominant
    (compiler/demo/matrix.py:64-80): the off-diagonal pattern stays, entries
    are divided by the largest magnitude, and ``a_ii = 1 + sum_j |a_ij|``."""
    matrix = sp.csr_matrix(matrix, dtype=np.float64, copy=True)
    matrix.sum_duplicates()
    matrix.eliminate_zeros()
    if not matrix.nnz:
        raise ValueError("Matrix Market sample is empty.")
    scale = float(np.max(np.abs(matrix.data)))
    if scale:
        matrix.data /= scale
    coo = matrix.tocoo()
    off = coo.row != coo.col
    n = matrix.shape[0]
    row_sum = np.bincount(coo.row[off], weights=np.abs(coo.data[off]),
                          minlength=n)
    rows = np.concatenate((coo.row[off], np.arange(n)))
    cols = np.concatenate((coo.col[off], np.arange(n)))
    data = np.concatenate((coo.data[off], row_sum + 1.0))
    result = sp.coo_matrix((data, (rows, cols)), shape=matrix.shape).tocsr()
    result.sort_indices()
    return result


def load_matrix_market(matrix_path, max_size=DEFAULT_MAX_N):
    """Load and regularise a square real Matrix Market input; ``max_size``
    keeps the leading principal block (0 = the whole matrix), as
    compiler/demo/matrix.py:26-62."""
    if max_size < 0:
        raise ValueError("max_size must be nonnegative.")
    matrix = read_matrix_market(matrix_path)
    if matrix.shape[0] != matrix.shape[1]:
        raise ValueError(
            f"Matrix Market input must be square, got {matrix.shape}.")
    if max_size:
        size = min(max_size, matrix.shape[0])
        matrix = matrix[:size, :size]
    return regularize(matrix)


def lower_triangle(matrix, storage):
    """The lower triangle (diagonal included) as ``(indptr, indices, data)``
    int32/int32/float64 arrays with sorted indices: CSR has the diagonal last
    in every row, CSC first in every column -- the layouts the SpTRSV loops
    assume (compiler/demo/sptrsv.py:26-43, README.md:85-92)."""
    lower = sp.tril(matrix, format="csr")
    if storage == "csr":
        out = sp.csr_matrix(lower)
    elif storage == "csc":
        out = sp.csc_matrix(lower)
    else:
        raise ValueError("storage must be 'csr' or 'csc'.")
    out.sort_indices()
    return (out.indptr.astype(np.int32), out.indices.astype(np.int32),
            out.data.astype(np.float64))


def manufactured_rhs(indptr, indices, data, storage):
    """``b = L @ linspace(1, 2, n)`` (compiler/demo/sptrsv.py:51-52)."""
    n = len(indptr) - 1
    kind = sp.csr_matrix if storage == "csr" else sp.csc_matrix
    lower = kind((data, indices, indptr), shape=(n, n))
    expected = np.linspace(1.0, 2.0, n)
    return np.asarray(lower @ expected).ravel(), expected

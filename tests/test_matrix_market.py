"""Matrix Market ingestion and the regulariser (host code, no GPU), and the
demo entry point on a generated file (GPU)."""

import gzip

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp
from scipy.sparse.linalg import spsolve_triangular

from lcd_amd.demo import matrix as M


def random_sparse(n, density, seed, symmetric=False):
    rng = np.random.default_rng(seed)
    a = sp.random(n, n, density=density, random_state=rng, format="coo")
    a.data = rng.uniform(-3.0, 3.0, a.nnz)
    if symmetric:
        a = sp.tril(a) + sp.tril(a, -1).T
    return sp.csr_matrix(a)


@pytest.mark.parametrize("symmetry", ["general", "symmetric", "skew-symmetric"])
@pytest.mark.parametrize("field", ["real", "integer", "pattern"])
def test_coordinate_reader_matches_scipy(tmp_path, symmetry, field):
    if field == "pattern" and symmetry == "skew-symmetric":
        pytest.skip("not a Matrix Market combination")
    a = random_sparse(40, 0.08, 5)
    if symmetry == "symmetric":
        a = sp.csr_matrix(sp.tril(a) + sp.tril(a, -1).T)
    elif symmetry == "skew-symmetric":
        a = sp.csr_matrix(sp.tril(a, -1) - sp.tril(a, -1).T)
    if field == "integer":
        a.data = np.round(a.data * 3)
    elif field == "pattern":
        a.data[:] = 1.0
    a.eliminate_zeros()
    path = tmp_path / "a.mtx"
    scipy.io.mmwrite(str(path), a, field=field, symmetry=symmetry,
                     comment="generated\nfor the reader test")
    mine = M.read_matrix_market(path)
    theirs = sp.csr_matrix(scipy.io.mmread(str(path)))
    assert mine.shape == theirs.shape
    assert (mine != theirs).nnz == 0
    np.testing.assert_array_equal(mine.toarray(), theirs.toarray())


def test_array_format_gzip_and_duplicates(tmp_path):
    rng = np.random.default_rng(2)
    dense = rng.normal(size=(6, 6))
    path = tmp_path / "d.mtx"
    scipy.io.mmwrite(str(path), dense)
    np.testing.assert_array_equal(M.read_matrix_market(path).toarray(), dense)
    symmetric = dense + dense.T
    scipy.io.mmwrite(str(path), symmetric, symmetry="symmetric")
    np.testing.assert_array_equal(M.read_matrix_market(path).toarray(), symmetric)
    text = ("%%MatrixMarket matrix coordinate real general\n% c\n\n3 3 4\n"
            "1 1 2.0\n2 1 -1.5\n2 1 0.5\n3 3 1e0\n")
    zipped = tmp_path / "z.mtx.gz"
    with gzip.open(zipped, "wt") as handle:
        handle.write(text)
    got = M.read_matrix_market(zipped).toarray()
    np.testing.assert_array_equal(
        got, np.array([[2.0, 0, 0], [-1.0, 0, 0], [0, 0, 1.0]]))


def test_reader_errors(tmp_path):
    path = tmp_path / "bad.mtx"
    path.write_text("%%MatrixMarket matrix coordinate complex general\n1 1 1\n1 1 1 0\n")
    with pytest.raises(M.MatrixMarketError, match="Complex"):
        M.read_matrix_market(path)
    path.write_text("hello\n")
    with pytest.raises(M.MatrixMarketError, match="Not a Matrix Market"):
        M.read_matrix_market(path)
    path.write_text("%%MatrixMarket matrix coordinate real general\n2 2 1\n3 1 1.0\n")
    with pytest.raises(M.MatrixMarketError, match="outside"):
        M.read_matrix_market(path)
    path.write_text("%%MatrixMarket matrix coordinate real general\n2 3 1\n1 1 1.0\n")
    with pytest.raises(ValueError, match="square"):
        M.load_matrix_market(path)
    with pytest.raises(FileNotFoundError):
        M.read_matrix_market(tmp_path / "missing.mtx")
    with pytest.raises(ValueError, match="nonnegative"):
        M.load_matrix_market(path, max_size=-1)


def test_regulariser_definition(tmp_path):
    """Dense restatement: scale by max |a|, drop the diagonal, then
    a_ii = 1 + sum_j |a_ij| (compiler/demo/matrix.py:64-80)."""
    a = random_sparse(30, 0.15, 9)
    path = tmp_path / "a.mtx"
    scipy.io.mmwrite(str(path), a)
    for size in (0, 12):
        dense = a.toarray()
        if size:
            dense = dense[:size, :size]
        dense = dense / np.abs(dense).max()
        np.fill_diagonal(dense, 0.0)
        np.fill_diagonal(dense, np.abs(dense).sum(axis=1) + 1.0)
        got = M.load_matrix_market(path, max_size=size)
        assert got.has_sorted_indices
        np.testing.assert_allclose(got.toarray(), dense, rtol=0, atol=1e-15)
        # strictly diagonally dominant, every diagonal entry stored
        assert np.all(got.diagonal() >= 1.0)
    for storage in ("csr", "csc"):
        indptr, indices, data = M.lower_triangle(got, storage)
        assert indptr.dtype == np.int32 and indices.dtype == np.int32
        n = len(indptr) - 1
        diagonal = indptr[1:] - 1 if storage == "csr" else indptr[:-1]
        np.testing.assert_array_equal(indices[diagonal], np.arange(n))
        rhs, expected = M.manufactured_rhs(indptr, indices, data, storage)
        kind = sp.csr_matrix if storage == "csr" else sp.csc_matrix
        lower = kind((data, indices, indptr), shape=(n, n))
        np.testing.assert_allclose(
            spsolve_triangular(sp.csr_matrix(lower), rhs, lower=True),
            expected, rtol=1e-12)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["wavefront", "sync_free"])
def test_demo_on_a_matrix_market_file(tmp_path, mode):
    from lcd_amd.demo import sptrsv
    a = random_sparse(900, 0.01, 4, symmetric=True)
    path = tmp_path / "sym.mtx"
    scipy.io.mmwrite(str(path), a, symmetry="symmetric")
    results = sptrsv.run_demo(path, max_size=0, storage="both",
                              verbose=False, execution_mode=mode)
    assert set(results) == {"csr", "csc"}
    for result, error in results.values():
        assert result.shape == (900,)
        assert error <= 1e-12
    sample = sptrsv.run_demo(path, max_size=100, storage="csc", verbose=False,
                             execution_mode=mode)
    assert sample["csc"][0].shape == (100,) and sample["csc"][1] <= 1e-12


@pytest.mark.gpu
def test_ilu0_demo_on_a_matrix_market_file(tmp_path):
    from lcd_amd.demo import spilu0
    a = random_sparse(300, 0.03, 8, symmetric=True)
    path = tmp_path / "ilu.mtx"
    scipy.io.mmwrite(str(path), a, symmetry="symmetric")
    for mode in ("wavefront", "sync_free"):
        factor, error = spilu0.run_demo(path, max_size=0, execution_mode=mode,
                                        verbose=False)
        assert factor.shape == (M.load_matrix_market(path, 0).nnz,)
        assert error <= 1e-12


def test_matrix_list_orders_by_declared_entry_count(tmp_path):
    from lcd_amd.demo import matrix_bench
    sizes = {"big.mtx": (60, 0.2), "small.mtx": (30, 0.05), "mid.mtx": (50, 0.1)}
    for seed, (name, (n, density)) in enumerate(sizes.items()):
        scipy.io.mmwrite(str(tmp_path / name), random_sparse(n, density, seed),
                         comment="generated")
    (tmp_path / "list.txt").write_text("big.mtx\nsmall.mtx\n\nmid.mtx\n")
    ordered = matrix_bench.matrix_list(tmp_path / "list.txt", str(tmp_path))
    assert [p.split("/")[-1] for p in ordered] == [
        "small.mtx", "mid.mtx", "big.mtx"]


@pytest.mark.gpu
def test_matrix_list_benchmark(tmp_path):
    """The list driver: every kernel on every listed matrix, results checked
    against the manufactured solution / the exact-ILU0 pattern identity."""
    import io
    from lcd_amd.demo import matrix_bench
    for seed, n in enumerate((400, 150)):
        scipy.io.mmwrite(str(tmp_path / f"m{n}.mtx"),
                         random_sparse(n, 0.02, 30 + seed, symmetric=True),
                         symmetry="symmetric")
    (tmp_path / "list.txt").write_text("m400.mtx\nm150.mtx\n")
    out = io.StringIO()
    rows = matrix_bench.run(tmp_path / "list.txt", str(tmp_path), warmup=1,
                            repeats=3, out=out)
    assert [row["matrix"] for row in rows] == ["m150.mtx"] * 3 + ["m400.mtx"] * 3
    assert [row["kernel"] for row in rows[:3]] == list(matrix_bench.KERNELS)
    for row in rows:
        assert row["max_abs_error"] <= 1e-11, row
        assert row["median_ms"] > 0 and row["levels"] >= 1
        assert row["p20_ms"] <= row["median_ms"] <= row["p80_ms"]
    lines = out.getvalue().strip().splitlines()
    assert lines[0].split(",") == list(matrix_bench.COLUMNS)
    assert len(lines) == 7

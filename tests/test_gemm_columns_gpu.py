"""Column remainder on the MI355X: an output N = 256 q + r wide (0 < r <= 64)
whose last r columns would cost the large tiles a round of their own runs as
two launches: the first 256 q columns on the large tiles, the last r on the
row kernel (r <= 8 with a K-major A: one wave per output row, no partial
sums) or on the thin 256x64 tile, which splits K when it fills few CUs.  With
split K off, the large-tile window and a thin-tile remainder are
bit-identical to the GEMM of A with that window's columns of B (same tiles'
K order); the row kernel sums K in its own fixed order and is checked
against the float64 oracle and for repeatability (fp32 storage within 1e-5
relative Frobenius error, bf16 storage within 1e-2)."""
import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 1e-2
# (m, k, n): the ragged config-2 shape and a wide output whose 256x256 grid
# just overflows 256 CUs (8 x 33 tiles)
SHAPES = [(4095, 1000, 4097), (2048, 300, 8193)]


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


def _columns(b, k, n, c0, c1, tb):
    """Columns [c0, c1) of B (k x n, or n x k when tb) as their own matrix."""
    return (b.reshape(n, k)[c0:c1] if tb else b.reshape(k, n)[:, c0:c1]).ravel().copy()


@pytest.mark.parametrize("m,k,n", SHAPES + [(2048, 640, 8192 + 40)])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, False)])
def test_windows_equal_their_own_products(amd, monkeypatch, m, k, n, dtype, ta, tb):
    monkeypatch.setenv("QUTAI_AMD_SPLITK", "1")
    a, b = normal(60 + n % 7, m * k, k ** -0.5), normal(70 + n % 5, k * n, k ** -0.5)
    left = upload(a, dtype)
    right = upload(b, dtype)
    got = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb)).reshape(m, n)
    main, r = n - n % 256, n % 256
    for c0, c1 in ((0, main), (main, n)):
        part = download(amd.gemm(left, upload(_columns(b, k, n, c0, c1, tb), dtype), m, k, c1 - c0,
                                 transpose_left=ta, transpose_right=tb)).reshape(m, c1 - c0)
        if c0 == main and r <= 8 and not ta:  # the row kernel: its own K order
            exact = ora.gemm_f64(stored(a, dtype), stored(_columns(b, k, n, c0, c1, tb), dtype), m, k, c1 - c0,
                                 transpose_left=ta, transpose_right=tb)
            assert ora.rel_frobenius(got[:, c0:c1], exact) <= FP32_TOL
            again = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb)).reshape(m, n)
            assert np.array_equal(again, got)
        else:
            assert np.array_equal(got[:, c0:c1], part), (c0, c1)


@pytest.mark.parametrize("m,k,n", SHAPES + [(2048, 640, 8192 + 40)])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_remainder_matches_oracle(amd, m, k, n, dtype):
    """Default path: the row kernel for the first two shapes, the thin tile
    in ten K chunks for the 40-column remainder."""
    a, b = normal(80, m * k, k ** -0.5), normal(81, k * n, k ** -0.5)
    left, right = upload(a, dtype), upload(b, dtype)
    sa, sb = stored(a, dtype), stored(b, dtype)
    rows = sorted({0, 1, m // 2, m - 1, *np.random.default_rng(9).choice(m, 10, replace=False).tolist()})
    exact = ora.gemm_f64(sa, sb, m, k, n, row_list=rows)
    got = download(amd.gemm(left, right, m, k, n)).reshape(m, n)
    assert ora.rel_frobenius(got[rows], exact) <= FP32_TOL
    tail = n - n % 256
    assert ora.rel_frobenius(got[rows][:, tail:], exact[:, tail:]) <= FP32_TOL
    rounded = download(amd.gemm(left, right, m, k, n, out_dtype="bfloat16")).reshape(m, n)
    assert ora.rel_frobenius(rounded[rows], exact) <= BF16_TOL
    # accumulate into an existing output: old + product, both windows
    start = normal(82, m * n)
    out = upload(start, "float32")
    amd.gemm(left, right, m, k, n, out=out, accumulate=True)
    expected = start.reshape(m, n)[rows].astype(np.float64) + exact
    assert ora.rel_frobenius(download(out).reshape(m, n)[rows], expected) <= FP32_TOL


@pytest.mark.parametrize("ta,tb", [(False, False), (False, True), (True, True)])
def test_remainder_mixed_inputs_autocast_and_bf16_accumulate(amd, ta, tb):
    """The remainder windows with fp32 A and bf16 B (mixed inputs take the bf16
    path: A is narrowed, B re-laid out first), the transpose forms the two
    remainder kernels take (row kernel for K-major A, thin tile otherwise),
    and a bf16 output accumulated in place: old + product rounded once."""
    m, k, n = 4095, 1000, 4097
    a, b = normal(90, m * k, k ** -0.5), normal(91, k * n, k ** -0.5)
    left, right = upload(a, "float32"), upload(b, "bfloat16")
    sa, sb = stored(a, "bfloat16"), stored(b, "bfloat16")  # the bf16 path rounds A once
    rows = sorted({0, 17, m // 3, m - 1, *np.random.default_rng(10).choice(m, 8, replace=False).tolist()})
    exact = ora.gemm_f64(sa, sb, m, k, n, transpose_left=ta, transpose_right=tb, row_list=rows)
    got = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb)).reshape(m, n)
    assert ora.rel_frobenius(got[rows], exact) <= FP32_TOL
    assert ora.rel_frobenius(got[rows][:, n - 1:], exact[:, n - 1:]) <= FP32_TOL
    start = normal(92, m * n)
    out = upload(start, "bfloat16")
    amd.gemm(left, right, m, k, n, out=out, accumulate=True, out_dtype="bfloat16", transpose_left=ta,
             transpose_right=tb)
    fp32 = got.astype(np.float32)
    want = stored(stored(start, "bfloat16").reshape(m, n).astype(np.float32) + fp32, "bfloat16")
    assert np.array_equal(download(out).reshape(m, n), want)

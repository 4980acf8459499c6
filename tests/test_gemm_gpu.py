"""GEMM parity on the MI355X through the amd backend (C ABI underneath).

Mirrors the reference GEMM contract tests (tests/test_gemm_precision.py,
cited per test) and checks BASELINE configs 1 and 2 against the float64
oracle on identical inputs: fp32 storage within 1e-5 relative Frobenius
error, bf16 storage (fp32 accumulation) within 1e-2.
"""
import math
import random

import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5   # fp32 storage vs float64 oracle (relative Frobenius)
BF16_TOL = 1e-2   # bf16 storage with fp32 accumulation vs float64 oracle


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


def bf16(value):
    return ora.bf16(value)


def max_abs(actual, expected):
    return max((abs(a - b) for a, b in zip(actual, expected)), default=0.0)


def reference(a, b, m, k, n, ta=False, tb=False):
    return ora.gemm(a, b, m, k, n, transpose_left=ta, transpose_right=tb)


# ---- Tensor @ on the fp32 path --------------------------------

def test_config1_tensor_matmul_matches_cpu_float64():
    from qutai_amd import Tensor

    rng = random.Random(0)
    a = [rng.uniform(-1, 1) for _ in range(128 * 256)]
    b = [rng.uniform(-1, 1) for _ in range(256 * 64)]
    expected = ora.matmul(a, b, (128, 256), (256, 64))  # the reference CPU float64 path
    left = Tensor(a, shape=(128, 256), device="amd", dtype="float32")
    right = Tensor(b, shape=(256, 64), device="amd", dtype="float32")
    result = left @ right
    assert result.shape == (128, 64) and result.dtype == "float32"
    got = np.array(result.storage.tolist())
    assert ora.rel_frobenius(got, expected) <= FP32_TOL


# ---- reference contract tests (tests/test_gemm_precision.py) -----------------------

def test_mixed_inputs_all_transposes_outside_autocast(amd):
    # tests/test_gemm_precision.py:35-56
    m, k, n = 5, 35, 17
    a = [math.sin(i * 0.17) for i in range(m * k)]
    b = [math.cos(i * 0.13) for i in range(k * n)]
    expected_a, expected_b = list(map(bf16, a)), list(map(bf16, b))
    runtime = amd.get_runtime()
    for da, db in (("bfloat16", "float32"), ("float32", "bfloat16"), ("bfloat16", "bfloat16")):
        left, right = amd.storage(a, dtype=da), amd.storage(b, dtype=db)
        assert left.nbytes == len(a) * (2 if da == "bfloat16" else 4)
        for ta, tb in ((False, False), (True, False), (False, True), (True, True)):
            before = runtime.mfma_launches
            result = amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb)
            assert result.dtype == "float32"
            assert runtime.mfma_launches == before + 1
            assert max_abs(result.tolist(), reference(expected_a, expected_b, m, k, n, ta, tb)) <= 4e-6


def test_bf16_output_and_in_place_accumulation(amd):
    # tests/test_gemm_precision.py:58-84
    m, k, n = 17, 35, 19
    a = [math.sin(i * 0.17) for i in range(m * k)]
    b = [math.cos(i * 0.13) for i in range(k * n)]
    left, right = amd.storage(a, dtype="bfloat16"), amd.storage(b, dtype="float32")
    expected = reference(list(map(bf16, a)), list(map(bf16, b)), m, k, n)
    target = amd.full(m * n, 0.25, dtype="float32")
    pointer = target.ptr
    result = amd.gemm(left, right, m, k, n, out=target)
    assert result is target and target.ptr == pointer
    assert max_abs(target.tolist(), expected) <= 4e-6
    amd.gemm(left, right, m, k, n, out=target, accumulate=True)
    assert max_abs(target.tolist(), [2 * x for x in expected]) <= 8e-6
    rounded = amd.gemm(left, right, m, k, n, out_dtype="bfloat16")
    assert rounded.nbytes == m * n * 2
    assert max_abs(rounded.tolist(), list(map(bf16, expected))) == 0
    old = rounded.tolist()
    amd.gemm(left, right, m, k, n, out_dtype="bfloat16", out=rounded, accumulate=True)
    assert max_abs(rounded.tolist(), [bf16(x + y) for x, y in zip(old, expected)]) == 0


def test_batch_broadcast_and_zero_inner(amd):
    # tests/test_gemm_precision.py:86-96
    left = amd.storage([1, 2, 3, 4, 5, 6], dtype="bfloat16")
    right = amd.storage([1, 2, 3, 4, 5, 6, 6, 5, 4, 3, 2, 1], dtype="float32")
    result = amd.gemm(left, right, 2, 3, 2, batch=2, left_stride=0)
    assert result.tolist() == [22, 28, 49, 64, 20, 14, 56, 41]
    empty = amd.storage([], dtype="bfloat16")
    target = amd.full(6, 3, dtype="float32")
    amd.gemm(empty, empty, 2, 0, 3, out=target, accumulate=True)
    assert target.tolist() == [3] * 6
    amd.gemm(empty, empty, 2, 0, 3, out=target)
    assert target.tolist() == [0] * 6


def test_autocast_and_fp64_compatibility(amd):
    # tests/test_gemm_precision.py:98-124
    from qutai_amd.backends.precision import set_matmul_precision

    for dtype in ("float32", "float64"):
        a = amd.storage([0.1, 0.2, 0.3, 0.4], dtype=dtype)
        with set_matmul_precision("bfloat16"):
            result = amd.gemm(a, a, 2, 2, 2)
        values = [bf16(x) for x in [0.1, 0.2, 0.3, 0.4]] if dtype == "float32" else [0.1, 0.2, 0.3, 0.4]
        assert result.dtype == dtype
        assert max_abs(result.tolist(), reference(values, values, 2, 2, 2)) <= (1e-7 if dtype == "float32" else 1e-15)
    a = amd.storage([0.1, 0.2, 0.3, 0.4], dtype="float32")
    result = amd.gemm(a, a, 2, 2, 2, out_dtype="bfloat16")
    expected = list(map(bf16, reference([0.1, 0.2, 0.3, 0.4], [0.1, 0.2, 0.3, 0.4], 2, 2, 2)))
    assert max_abs(result.tolist(), expected) == 0


def test_invalid_output_and_alias(amd):
    # tests/test_gemm_precision.py:126-137
    a = amd.full(4, 1, dtype="float32")
    for kwargs in ({"out": a}, {"accumulate": True}, {"out": amd.full(4, 0, dtype="bfloat16")},
                   {"left_stride": -1}):
        with pytest.raises(ValueError):
            amd.gemm(a, a, 2, 2, 2, **kwargs)
    with pytest.raises(ValueError):
        amd.gemm(a, a, 3, 2, 2)


def test_large_mixed_transposes_and_partial_output_tiles(amd):
    # tests/test_gemm_precision.py:139-189
    m, k, n = 1025, 129, 1025
    a = np.array([math.sin(i * 0.013) * 0.03 for i in range(m * k)])
    b = np.array([math.cos(i * 0.017) * 0.02 for i in range(k * n)])
    left, right = upload(a, "bfloat16"), upload(b, "float32")
    ra, rb = stored(a, "bfloat16"), stored(b, "bfloat16")
    coordinates = [0, 15, 16, 63, 64, 127, 128, 1023, 1024]
    for ta, tb in ((False, False), (True, False), (False, True), (True, True)):
        expected = ora.gemm_f64(ra, rb, m, k, n, transpose_left=ta, transpose_right=tb, row_list=coordinates)
        expected = expected[:, coordinates]
        target = amd.full(m * n, 0.25, dtype="float32")
        result = amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb, out=target)
        assert result is target
        got = download(target).reshape(m, n)[np.ix_(coordinates, coordinates)]
        assert np.abs(got - expected).max() <= 2e-7
        amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb, out=target, accumulate=True)
        got = download(target).reshape(m, n)[np.ix_(coordinates, coordinates)]
        assert np.abs(got - 2 * expected).max() <= 4e-7
    rounded = amd.gemm(left, right, m, k, n, out_dtype="bfloat16")
    assert rounded.nbytes == m * n * 2
    expected = ora.gemm_f64(ra, rb, m, k, n, row_list=coordinates)[:, coordinates]
    got = download(rounded).reshape(m, n)[np.ix_(coordinates, coordinates)]
    assert np.abs(got - ora.bf16_round_array(expected.astype(np.float32))).max() <= 6.2e-5


def test_long_reduction_partial_tiles_batch_and_accumulate(amd):
    # tests/test_gemm_precision.py:191-206 (exact closed form)
    m, k, n = 129, 8193, 1025
    left = amd.full(m * k, 0.5, dtype="bfloat16")
    right = upload(np.concatenate([np.full(k * n, -0.25), np.full(k * n, 0.5)]), "float32")
    target = amd.full(2 * m * n, 0.25, dtype="float32")
    result = amd.gemm(left, right, m, k, n, batch=2, left_stride=0, out=target, accumulate=True)
    assert result is target
    values = download(result)
    assert (values[: m * n] == -k * 0.125 + 0.25).all()
    assert (values[m * n:] == k * 0.25 + 0.25).all()


# ---- parity sweep against the float64 oracle ------------------------------------------

SHAPES = [(1, 1, 1), (7, 3, 5), (33, 17, 65), (64, 64, 64), (96, 200, 130), (257, 513, 129), (300, 64, 2000),
          (2000, 40, 48), (512, 1000, 384)]


@pytest.mark.parametrize("m,k,n", SHAPES)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_parity_all_transposes(amd, m, k, n, dtype):
    a = normal(100 + m, m * k)
    b = normal(200 + n, k * n)
    left, right = upload(a, dtype), upload(b, dtype)
    sa, sb = stored(a, dtype), stored(b, dtype)
    for ta in (False, True):
        for tb in (False, True):
            exact = ora.gemm_f64(sa, sb, m, k, n, transpose_left=ta, transpose_right=tb)
            result = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb)).reshape(m, n)
            # fp32 accumulation of exactly stored inputs: fp32-level agreement
            assert ora.rel_frobenius(result, exact) <= FP32_TOL
            if dtype == "bfloat16":
                unrounded = ora.gemm_f64(a.astype(np.float64), b.astype(np.float64), m, k, n,
                                         transpose_left=ta, transpose_right=tb)
                assert ora.rel_frobenius(result, unrounded) <= BF16_TOL
            rounded = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb,
                                        out_dtype="bfloat16")).reshape(m, n)
            assert ora.rel_frobenius(rounded, exact) <= BF16_TOL


def test_strided_batch_and_broadcast(amd):
    batch, m, k, n = 5, 70, 90, 110
    a = normal(1, batch * m * k)
    b = normal(2, k * n)
    for dtype in ("float32", "bfloat16"):
        left, right = upload(a, dtype), upload(b, dtype)
        result = download(amd.gemm(left, right, m, k, n, batch=batch, right_stride=0)).reshape(batch, m, n)
        sa, sb = stored(a, dtype).reshape(batch, m * k), stored(b, dtype)
        for z in range(batch):
            exact = ora.gemm_f64(sa[z], sb, m, k, n)
            assert ora.rel_frobenius(result[z], exact) <= FP32_TOL


def test_results_are_deterministic(amd):
    a, b = normal(3, 1000 * 777), normal(4, 777 * 900)
    for dtype in ("float32", "bfloat16"):
        left, right = upload(a, dtype), upload(b, dtype)
        first = download(amd.gemm(left, right, 1000, 777, 900))
        for _ in range(2):
            assert np.array_equal(download(amd.gemm(left, right, 1000, 777, 900)), first)


# ---- BASELINE config 2 at full size ------------------------------------------------

def sampled_rows(m, count=48, seed=0):
    rows = {0, 1, m // 2, m - 1}
    rows.update(np.random.default_rng(seed).choice(m, size=count, replace=False).tolist())
    return sorted(rows)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_config2_square_4096(amd, dtype):
    m = k = n = 4096
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(m * k) * k ** -0.5).astype(np.float32)
    b = (rng.standard_normal(k * n) * k ** -0.5).astype(np.float32)
    left, right = upload(a, dtype), upload(b, dtype)
    result = download(amd.gemm(left, right, m, k, n)).reshape(m, n)
    rows = sampled_rows(m)
    exact_stored = ora.gemm_f64(stored(a, dtype), stored(b, dtype), m, k, n, row_list=rows)
    exact_unrounded = ora.gemm_f64(a.astype(np.float64), b.astype(np.float64), m, k, n, row_list=rows)
    assert ora.rel_frobenius(result[rows], exact_stored) <= FP32_TOL
    assert ora.rel_frobenius(result[rows], exact_unrounded) <= (FP32_TOL if dtype == "float32" else BF16_TOL)
    assert np.isfinite(result).all()


@pytest.mark.parametrize("order", ["MxNxK", "MxKxN"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_config2_ragged_edge_shape(amd, order, dtype):
    # 4095 x 4097 x 1000 read both ways (rows, cols, inner) and (rows, inner, cols)
    m, n, k = (4095, 4097, 1000) if order == "MxNxK" else (4095, 1000, 4097)
    rng = np.random.default_rng(1)
    a = (rng.standard_normal(m * k) * k ** -0.5).astype(np.float32)
    b = (rng.standard_normal(k * n) * k ** -0.5).astype(np.float32)
    left, right = upload(a, dtype), upload(b, dtype)
    result = download(amd.gemm(left, right, m, k, n)).reshape(m, n)
    rows = sampled_rows(m)
    exact = ora.gemm_f64(stored(a, dtype), stored(b, dtype), m, k, n, row_list=rows)
    assert ora.rel_frobenius(result[rows], exact) <= FP32_TOL
    unrounded = ora.gemm_f64(a.astype(np.float64), b.astype(np.float64), m, k, n, row_list=rows)
    assert ora.rel_frobenius(result[rows], unrounded) <= (FP32_TOL if dtype == "float32" else BF16_TOL)
    # the last column and row (tile tails) are checked element-wise
    assert np.abs(result[rows][:, -1] - exact[:, -1]).max() <= 1e-5 * np.abs(exact).max()

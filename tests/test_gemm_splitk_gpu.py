"""Split-K GEMM on the MI355X: K cut into chunks of a multiple of 64, fp32
partial products in the workspace, one ordered reduction.  Forced splits
(QUTAI_AMD_SPLITK) over every transpose form, both storages, bf16 output,
accumulation and strided batches, with K that is not a multiple of the chunk
or of 64; and the decoder head's dX shape (1024 x 2048 outputs, K = 32768),
which splits on its own, on sampled rows against the float64 oracle (fp32
storage within 1e-5 relative Frobenius error, bf16 storage within 1e-2)."""
import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import download, normal, stored, upload

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 1e-2


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


@pytest.mark.parametrize("splits", [2, 3, 7])
@pytest.mark.parametrize("m,k,n", [(33, 200, 65), (300, 1000, 257), (129, 4100, 96)])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_forced_split_all_transposes(amd, monkeypatch, splits, m, k, n, dtype):
    monkeypatch.setenv("QUTAI_AMD_SPLITK", str(splits))
    a, b = normal(10 + m, m * k), normal(20 + n, k * n)
    left, right = upload(a, dtype), upload(b, dtype)
    sa, sb = stored(a, dtype), stored(b, dtype)
    for ta in (False, True):
        for tb in (False, True):
            exact = ora.gemm_f64(sa, sb, m, k, n, transpose_left=ta, transpose_right=tb)
            got = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb)).reshape(m, n)
            assert ora.rel_frobenius(got, exact) <= FP32_TOL, (ta, tb)
            rounded = download(amd.gemm(left, right, m, k, n, transpose_left=ta, transpose_right=tb,
                                        out_dtype="bfloat16")).reshape(m, n)
            assert ora.rel_frobenius(rounded, exact) <= BF16_TOL, (ta, tb)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_forced_split_accumulate_and_batch(amd, monkeypatch, dtype):
    monkeypatch.setenv("QUTAI_AMD_SPLITK", "4")
    batch, m, k, n = 3, 70, 900, 110
    a, b = normal(1, batch * m * k), normal(2, k * n)
    left, right = upload(a, dtype), upload(b, dtype)
    sa, sb = stored(a, dtype).reshape(batch, m * k), stored(b, dtype)
    got = download(amd.gemm(left, right, m, k, n, batch=batch, right_stride=0)).reshape(batch, m, n)
    for z in range(batch):
        assert ora.rel_frobenius(got[z], ora.gemm_f64(sa[z], sb, m, k, n)) <= FP32_TOL
    # accumulate into an existing fp32 and bf16 output
    start = normal(3, m * n)
    for out_dtype, tol in (("float32", FP32_TOL), ("bfloat16", BF16_TOL)):
        out = upload(start, out_dtype)
        amd.gemm(left, right, m, k, n, out=out, accumulate=True, out_dtype=out_dtype)
        expected = stored(start, out_dtype).reshape(m, n) + ora.gemm_f64(sa[0], sb, m, k, n)
        assert ora.rel_frobenius(download(out).reshape(m, n), expected) <= tol


def test_split_results_are_repeatable(amd, monkeypatch):
    monkeypatch.setenv("QUTAI_AMD_SPLITK", "5")
    a, b = normal(5, 200 * 3000), normal(6, 3000 * 300)
    left, right = upload(a, "bfloat16"), upload(b, "bfloat16")
    first = download(amd.gemm(left, right, 200, 3000, 300))
    for _ in range(2):
        assert np.array_equal(download(amd.gemm(left, right, 200, 3000, 300)), first)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_decoder_head_shape_splits_by_itself(amd, dtype):
    m, k, n = 1024, 32768, 2048
    runtime = amd.get_runtime()
    ws = runtime.lib.qutai_amd_gemm_workspace_size(m, k, n, 1, 0, 0, 0, 0, 0 if dtype == "float32" else 5,
                                                   0 if dtype == "float32" else 5, 0)
    assert ws >= 2 * m * n * 4  # room for at least two fp32 partial products
    rng = np.random.default_rng(7)
    a = (rng.standard_normal(m * k) * k ** -0.5).astype(np.float32)
    b = (rng.standard_normal(k * n) * k ** -0.5).astype(np.float32)
    got = download(amd.gemm(upload(a, dtype), upload(b, dtype), m, k, n)).reshape(m, n)
    rows = sorted({0, 1, 511, 1023, *np.random.default_rng(8).choice(m, 12, replace=False).tolist()})
    exact = ora.gemm_f64(stored(a, dtype), stored(b, dtype), m, k, n, row_list=rows)
    assert ora.rel_frobenius(got[rows], exact) <= FP32_TOL
    assert np.isfinite(got).all()


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
@pytest.mark.parametrize("m,k,n,tb", [(8192, 2048, 8, True), (2000, 1500, 40, False), (48, 3000, 1024, False)])
def test_thin_outputs_split_by_themselves(amd, dtype, m, k, n, tb):
    """A router-shaped product (8192 x 2048 x 8, X W^T) and other thin outputs
    over few 256-wide blocks take K chunks without being forced: the
    workspace asks for fp32 partials, and every row matches the oracle."""
    runtime = amd.get_runtime()
    code = 0 if dtype == "float32" else 5
    ws = runtime.lib.qutai_amd_gemm_workspace_size(m, k, n, 1, 0, 0, 0, int(tb), code, code, 0)
    assert ws >= 2 * m * n * 4
    a, b = normal(40 + n, m * k), normal(50 + n, k * n)
    got = download(amd.gemm(upload(a, dtype), upload(b, dtype), m, k, n, transpose_right=tb)).reshape(m, n)
    exact = ora.gemm_f64(stored(a, dtype), stored(b, dtype), m, k, n, transpose_right=tb)
    assert ora.rel_frobenius(got, exact) <= FP32_TOL
    rounded = download(amd.gemm(upload(a, dtype), upload(b, dtype), m, k, n, transpose_right=tb,
                                out_dtype="bfloat16")).reshape(m, n)
    assert ora.rel_frobenius(rounded, exact) <= BF16_TOL

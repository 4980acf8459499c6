"""qutai_amd_gemm_static (the allocation-free GEMM entry point) called
through the C ABI against qutai_amd_gemm (the workspace-taking entry point
that amd.gemm drives): bit-identical outputs, two calls in a row with the
second on smaller operands, for each way the workspace is used (operand
narrowing under autocast, re-layout of a ragged operand, split-K partial
sums) and for operands used in place; an oversized request is refused
before anything is launched."""
import numpy as np
import pytest

from tests.helpers import download, normal, upload

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def amd():
    from qutai_amd.backends import amd as backend

    backend.get_runtime()
    return backend


def static_gemm(amd, a, b, rows, inner, cols, *, transpose_left=False, transpose_right=False, out_dtype="float32",
                bf16_compute=False, out=None):
    """One qutai_amd_gemm_static call through the C ABI."""
    runtime = amd.get_runtime()
    out = out if out is not None else amd.full(rows * cols, 0.0, dtype=out_dtype)
    runtime.call("qutai_amd_gemm_static", a.ptr, b.ptr, out.ptr, rows, inner, cols, 1, rows * inner, inner * cols,
                 int(transpose_left), int(transpose_right), amd.code(a.dtype), amd.code(b.dtype),
                 amd.code(out.dtype), 0, int(bf16_compute))
    return out


def reference_gemm(amd, a, b, rows, inner, cols, *, transpose_left=False, transpose_right=False,
                   out_dtype="float32", bf16_compute=False):
    from qutai_amd.backends.precision import set_matmul_precision

    with set_matmul_precision("bfloat16" if bf16_compute else None):
        return amd.gemm(a, b, rows, inner, cols, transpose_left=transpose_left, transpose_right=transpose_right,
                        out_dtype=out_dtype)


CASES = {
    # fp32 operands into the bf16 path (autocast): both narrowed into the scratch
    "autocast": [dict(shape=(1536, 1024, 2048), dtype="float32", bf16_compute=True),
                 dict(shape=(256, 512, 384), dtype="float32", bf16_compute=True)],
    # a 4097-wide row-major B: re-laid out with a 16-byte-aligned pitch
    "ragged": [dict(shape=(1000, 512, 4097), dtype="bfloat16"),
               dict(shape=(300, 256, 1001), dtype="bfloat16")],
    # few output tiles over a long K: split-K partial sums in the scratch
    "split_k": [dict(shape=(1024, 32768, 2048), dtype="bfloat16", out_dtype="bfloat16"),
                dict(shape=(512, 4096, 2048), dtype="bfloat16", transpose_left=True)],
    # aligned bf16 operands: used in place, no scratch
    "in_place": [dict(shape=(512, 768, 1024), dtype="bfloat16", transpose_right=True),
                 dict(shape=(128, 256, 64), dtype="bfloat16")],
    # column remainders: the row kernel's compact B columns (4097 = 16 x 256 + 1)
    # and the thin tile's K-chunk partials (8232 = 32 x 256 + 40) in the scratch
    "columns": [dict(shape=(4095, 1000, 4097), dtype="bfloat16"),
                dict(shape=(2048, 640, 8232), dtype="bfloat16")],
    # fp32 true-fp32 path with a split K
    "fp32_split": [dict(shape=(1024, 16384, 1024), dtype="float32"),
                   dict(shape=(256, 8192, 256), dtype="float32")],
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_static_entry_matches_workspace_entry(amd, name):
    for call, case in enumerate(CASES[name]):
        rows, inner, cols = case["shape"]
        ta, tb = case.get("transpose_left", False), case.get("transpose_right", False)
        x = normal(100 + call, (inner, rows) if ta else (rows, inner), inner ** -0.5)
        w = normal(200 + call, (cols, inner) if tb else (inner, cols))
        a, b = upload(x, case["dtype"]), upload(w, case["dtype"])
        kwargs = dict(transpose_left=ta, transpose_right=tb, out_dtype=case.get("out_dtype", "float32"),
                      bf16_compute=case.get("bf16_compute", False))
        print(f"case {name} call {call}: {rows}x{inner}x{cols} {case['dtype']}", flush=True)
        expected = download(reference_gemm(amd, a, b, rows, inner, cols, **kwargs))
        got = download(static_gemm(amd, a, b, rows, inner, cols, **kwargs))
        assert got.tobytes() == expected.tobytes(), f"{name} call {call}"
        assert np.isfinite(got).all()


def test_oversized_request_is_refused_before_launch(amd):
    """fp32 operands of 2 x 32 Mi elements into the bf16 path need 128 MiB of
    narrowed copies plus alignment slack: more than the scratch holds."""
    runtime = amd.get_runtime()
    capacity = runtime.lib.qutai_amd_gemm_static_capacity()
    assert capacity == 128 << 20
    rows, inner, cols = 4096, 8192, 4096
    a = amd.full(rows * inner, 1.0, dtype="float32")
    b = amd.full(inner * cols, 1.0, dtype="float32")
    out = amd.full(rows * cols, -7.0, dtype="float32")
    with pytest.raises(RuntimeError, match="scratch"):
        static_gemm(amd, a, b, rows, inner, cols, bf16_compute=True, out=out)
    sample = download(out)[:: 4096 * 64]
    assert (sample == -7.0).all()  # nothing ran
    # the same entry point still serves the next call
    small = static_gemm(amd, amd.full(64 * 64, 1.0, dtype="float32"), amd.full(64 * 64, 2.0, dtype="float32"), 64,
                        64, 64, bf16_compute=True)
    assert (download(small) == 128.0).all()

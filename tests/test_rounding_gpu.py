"""fp32 -> bf16 rounding on the device, bit for bit against the reference's
encoder rule (src/qutai/backends/cuda.py:98-101: round to nearest even, a NaN
becomes (bits >> 16) | 0x40), restated by ``oracle.reference.bf16_words``.

The device kernels round with gfx950's v_cvt_pk_bf16_f32, so these tests pin
that instruction to the rule: every special class (signed zeros, infinities,
NaN payloads with and without the quiet bit, denormals, round-to-even ties,
overflow to infinity) and a million random bit patterns through the cast
kernel, and the GEMM epilogue's bf16 output against the same GEMM's fp32
output rounded on the host (every tile sums K in the same order, so the two
differ only by the final rounding)."""
from array import array

import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import upload

pytestmark = pytest.mark.gpu

SPECIAL = np.array([
    0x00000000, 0x80000000, 0x7F800000, 0xFF800000,              # zeros, infinities
    0x7F800001, 0x7FA00000, 0xFFC00001, 0x7FFFFFFF, 0xFF812345,  # NaNs (signalling, quiet, payloads)
    0x7FC00000, 0xFFFFFFFF, 0x7F80FFFF, 0x7F817FFF,
    0x00000001, 0x80000001, 0x007FFFFF, 0x00008000, 0x00018000,  # denormals and denormal ties
    0x3F808000, 0x3F818000, 0x3F80FFFF, 0x3F807FFF,              # ties to even, just below / above
    0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F8000, 0x7F7F7FFF,              # overflow to infinity and the largest finite
], dtype=np.uint32)


def _bits_to_bf16_words(bits):
    from qutai_amd.backends import amd

    x = amd.storage(array("f", bits.astype(np.uint32).tobytes()), dtype="float32")
    y = amd.from_storage(x, dtype="bfloat16")
    return np.frombuffer(y.to_array(), dtype=np.uint16)


def test_cast_special_values_bit_exact():
    got = _bits_to_bf16_words(SPECIAL)
    want = ora.bf16_words(SPECIAL.view(np.float32))
    assert np.array_equal(got, want), [(hex(b), hex(g), hex(w)) for b, g, w in zip(SPECIAL, got, want) if g != w]


def test_cast_random_bit_patterns_bit_exact():
    bits = np.random.default_rng(11).integers(0, 2 ** 32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    got = _bits_to_bf16_words(bits)
    want = ora.bf16_words(bits.view(np.float32))
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, [(hex(bits[i]), hex(got[i]), hex(want[i])) for i in bad[:10]]


@pytest.mark.parametrize("m,k,n,ta,tb", [
    (512, 256, 384, False, False),   # whole tiles: straight-line epilogue
    (512, 256, 384, False, True),
    (300, 100, 260, False, False),   # ragged tiles: bounds-checked epilogue
    (300, 100, 262, True, False),    # odd pitch: 4-byte bf16 rows
    (300, 100, 261, False, False),   # odd element pitch: 2-byte bf16 rows, 4-byte fp32 rows
    (129, 64, 257, False, True),
])
def test_gemm_bf16_output_is_rounded_fp32_output(m, k, n, ta, tb):
    from qutai_amd.backends import amd

    rng = np.random.default_rng(m + n)
    a = upload(rng.standard_normal(m * k), "bfloat16")
    b = upload(rng.standard_normal(k * n), "bfloat16")
    kw = dict(transpose_left=ta, transpose_right=tb)
    wide = amd.gemm(a, b, m, k, n, out_dtype="float32", **kw)
    narrow = amd.gemm(a, b, m, k, n, out_dtype="bfloat16", **kw)
    got = np.frombuffer(narrow.to_array(), dtype=np.uint16)
    want = ora.bf16_words(np.frombuffer(wide.to_array(), dtype=np.float32))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("m,k,n", [(512, 256, 384), (300, 100, 264), (300, 100, 261)])
def test_gemm_accumulate_adds_old_value_before_one_rounding(m, k, n):
    """out = round(old + A@B) (gemm.cu:25-32) on whole tiles (straight-line
    epilogue) and ragged tiles: bit-exact against the fp32 product of the
    same GEMM added to the old values on the host."""
    from qutai_amd.backends import amd

    rng = np.random.default_rng(m * n)
    a = upload(rng.standard_normal(m * k), "bfloat16")
    b = upload(rng.standard_normal(k * n), "bfloat16")
    product = np.frombuffer(amd.gemm(a, b, m, k, n, out_dtype="float32").to_array(), dtype=np.float32)
    old = rng.standard_normal(m * n).astype(np.float32)
    wide = upload(old, "float32")
    amd.gemm(a, b, m, k, n, out=wide, accumulate=True)
    assert np.array_equal(np.frombuffer(wide.to_array(), dtype=np.float32), old + product)
    narrow = upload(old, "bfloat16")
    old16 = ora.bf16_values(np.frombuffer(narrow.to_array(), dtype=np.uint16)).astype(np.float32)
    amd.gemm(a, b, m, k, n, out=narrow, out_dtype="bfloat16", accumulate=True)
    assert np.array_equal(np.frombuffer(narrow.to_array(), dtype=np.uint16), ora.bf16_words(old16 + product))

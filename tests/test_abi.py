"""The C-ABI library loads and exports every entry point of include/qutai_amd.h.

Runs without a GPU: loading libqutai_amd.so links libamdhip64 but touches no
device; no compute entry point is called.
"""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "qutai_amd.h"
LIBRARY = ROOT / "qutai_amd" / "libqutai_amd.so"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:int|size_t|int64_t)\s+(qutai_amd_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_entry_points():
    names = declared_functions()
    assert "qutai_amd_gemm" in names and "qutai_amd_gemm_grouped" in names
    assert len(names) == len(set(names))


@pytest.mark.skipif(not LIBRARY.exists(), reason="libqutai_amd.so not built (python -m qutai_amd.build)")
def test_library_exports_every_declared_symbol():
    library = ctypes.CDLL(str(LIBRARY))
    missing = [name for name in declared_functions() if not hasattr(library, name)]
    assert not missing, missing


def test_python_binding_table_matches_the_header():
    from qutai_amd.backends import amd_runtime

    assert set(amd_runtime.SIGNATURES) == set(declared_functions())


@pytest.mark.skipif(not LIBRARY.exists(), reason="libqutai_amd.so not built")
def test_bindings_apply_without_a_device():
    from qutai_amd.backends import amd_runtime

    library = amd_runtime.load_library()
    # pure host helper: workspace sizing needs no GPU.  (rows, inner, cols,
    # batch, strides, ta, tb, a dtype, b dtype, bf16 compute)
    size = library.qutai_amd_gemm_workspace_size
    assert size(64, 64, 64, 1, 0, 0, 0, 0, 5, 5, 0) == 0  # aligned bf16 x bf16: in place
    # fp32 A into the bf16 path: a 64x64 bf16 copy (8 KiB, 256-byte rounded) + slack
    assert size(64, 64, 64, 1, 0, 0, 0, 0, 0, 5, 0) == 64 * 64 * 2 + 256
    # 4097-wide row-major bf16 B (NN): rows padded to 4104 elements
    assert size(8, 16, 4097, 1, 0, 0, 0, 0, 5, 5, 0) == (16 * 4104 * 2 + 255) // 256 * 256 + 256
    # fp32 x fp32 aligned: in place
    assert size(64, 64, 64, 1, 0, 0, 0, 0, 0, 0, 0) == 0
    # autocast of two fp32 operands: both copied
    assert size(64, 64, 64, 1, 0, 0, 0, 0, 0, 0, 1) == 2 * 64 * 64 * 2 + 256
    # split-K: 1024 x 2048 outputs over K = 32768 fill a quarter of the
    # 128x128-tile slots of 256 CUs (the count used without a device); bf16
    # then picks 256x256 tiles in eight K chunks of 4096 (32 tiles x 8 = one
    # round): eight fp32 partial products; fp32 keeps 128x128 in four chunks
    assert size(1024, 32768, 2048, 1, 0, 0, 0, 0, 5, 5, 0) == 8 * 1024 * 2048 * 4 + 256
    assert size(1024, 32768, 2048, 1, 0, 0, 0, 0, 0, 0, 0) == 4 * 1024 * 2048 * 4 + 256
    # K/V weight gradient shape: 128x128 tiles in four chunks of 1024
    assert size(512, 4096, 2048, 1, 0, 0, 1, 0, 5, 5, 0) == 4 * 512 * 2048 * 4 + 256
    assert size(4096, 4096, 4096, 1, 0, 0, 0, 0, 5, 5, 0) == 0  # a full round of tiles: no split
    # RMSNorm backward partial sums: one row of floats per 16 rows
    rms = library.qutai_amd_rms_norm_workspace
    assert rms(4096, 2048) == 256 * 2048 and rms(65, 8) == 5 * 8 and rms(0, 8) == 0


@pytest.mark.skipif(not LIBRARY.exists(), reason="libqutai_amd.so not built")
def test_argument_checks_reject_before_any_device_call():
    """Entry points validate on the host and return QA_EINVAL (-1) before
    they launch anything, so these calls with stand-in pointers never reach
    a device."""
    from qutai_amd.backends import amd_runtime

    library = amd_runtime.load_library()
    fake = 1 << 20  # a 16-byte aligned stand-in address, never dereferenced
    # grouped expert GEMM: a 256-row tile of a 2^23-wide bf16 operand spans
    # 2^32 bytes, beyond the 31-bit buffer descriptor range
    assert library.qutai_amd_gemm_grouped(fake, fake, fake, fake, 8, 512, 1 << 23, 64, 0, 1, 5, 5, 0, None, 0,
                                          None) == -1
    # gathered rows: the whole source matrix (2^19 rows of 2048 bf16 = 2^31
    # bytes) must stay inside one descriptor's 31-bit range
    assert library.qutai_amd_gemm_grouped(fake, fake, fake, fake, 8, 512, 2048, 64, 0, 1, 5, 5, 0, fake, 1 << 19,
                                          None) == -1
    assert library.qutai_amd_gemm_swiglu(fake, fake, fake, fake, None, None, fake, 8, 512, 2048, 64, 0, 5, fake,
                                         1 << 19, None) == -1
    # the pair form joins its two K halves at a multiple of 64
    assert library.qutai_amd_gemm_grouped_pair(fake, fake, fake, fake, fake, fake, 8, 512, 96, 64, 0, 0, 5, 0, 0,
                                               None) == -1
    # a gather needs the grouped form (offsets)
    assert library.qutai_amd_gemm_swiglu(fake, fake, fake, fake, None, None, None, 1, 512, 2048, 64, 0, 5, fake,
                                         16, None) == -1
    # strided copy: rank above 8, or an element size other than 2/4/8
    dims = (ctypes.c_int64 * 9)(*([2] * 9))
    assert library.qutai_amd_strided_copy(fake, fake, 9, dims, dims, dims, 4, None) == -1
    assert library.qutai_amd_strided_copy(fake, fake, 1, dims, dims, dims, 3, None) == -1
    # binary / unary op codes out of range; a backward without its gradient
    assert library.qutai_amd_binary(fake, fake, fake, 8, 4, 0, None, None) == -1
    assert library.qutai_amd_unary(fake, None, fake, 8, 14, 1.0, 0, None, None) == -1
    assert library.qutai_amd_unary(fake, None, fake, 8, 4, 0.0, 0, None, None) == -1
    # reduction over [outer][width][inner] needs inner >= 1 and a float dtype
    assert library.qutai_amd_reduce_sum(fake, fake, 1, 8, 0, 0, None, 0, None) == -1
    assert library.qutai_amd_reduce_sum(fake, fake, 1, 8, 1, 4, None, 0, None) == -1


@pytest.mark.skipif(not LIBRARY.exists(), reason="libqutai_amd.so not built")
def test_reduction_workspace_plan():
    """Long sums split into parts whose fp32 partials need a workspace; short
    or plentiful sums run in one pass."""
    from qutai_amd.backends import amd_runtime

    size = amd_runtime.load_library().qutai_amd_reduce_sum_workspace_size
    assert size(4096, 2048, 1, 0) == 0  # 4096 rows: one wave per row is enough
    assert size(1, 1 << 22, 1, 0) == 1024 * 4  # one long row: 1024 parts of 4096
    assert size(1, 1 << 22, 1, 1) == 1024 * 8  # fp64 partials
    assert size(1, 4096, 2048, 0) == 32 * 2048 * 4  # 2048 columns of 4096: 32 parts of 128
    assert size(4, 100, 1, 0) == 0

"""Every bf16 GEMM tile shape (256x256, 192x256, 256x192, 256x128, 128x128 with
a four- or two-stage ring, the thin 256x64 and 64x256 tiles, the 256x256
ping-pong kernel for K a multiple of 64, and the short-K row strips of NT
products with K <= 64 and N a multiple of 16), and every fp32 tile,
sums K in the same order, in chunks of 64 through the same MFMA chain, so a
tile forced with QUTAI_AMD_GEMM_TILE gives bit-identical output to any other
for the same call: whole and ragged tiles, the four transpose forms, fp32 and
bf16 output, accumulation and a strided batch.  The variable is read once per
process, so each tile runs in a child process that writes its outputs to a
file; the 256x256 outputs are also checked against the float64 oracle
(bf16 storage within 1e-2 relative Frobenius error, the reference's bar)."""
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from oracle import reference as ora
from tests.helpers import normal, stored

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
CASES = [(700, 320, 600, 1), (384, 256, 512, 1), (200, 130, 70, 3), (1024, 192, 768, 2), (700, 64, 600, 2),
         (129, 40, 257, 1), (320, 64, 1040, 3), (129, 24, 144, 2), (64, 8, 2064, 1), (129, 128, 70, 2)]

CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[2])
from qutai_amd.backends import amd
from tests.helpers import download, normal, upload
cases = eval(sys.argv[3])
dtype = sys.argv[4] if len(sys.argv) > 4 else "bfloat16"
outs = {}
for m, k, n, batch in cases:
    a, b = normal(10 + m, batch * m * k), normal(20 + n, batch * k * n)
    left, right = upload(a, dtype), upload(b, dtype)
    for ta in (False, True):
        for tb in (False, True):
            kw = dict(batch=batch, transpose_left=ta, transpose_right=tb)
            for od in ("float32", "bfloat16"):
                outs[f"{m}_{k}_{n}_{batch}_{ta:d}{tb:d}_{od}"] = download(amd.gemm(left, right, m, k, n, out_dtype=od, **kw))
            acc = upload(normal(30 + m, batch * m * n), "bfloat16")
            amd.gemm(left, right, m, k, n, out=acc, out_dtype="bfloat16", accumulate=True, **kw)
            outs[f"{m}_{k}_{n}_{batch}_{ta:d}{tb:d}_acc"] = download(acc)
# large outputs (the ragged config-2 shape) are compared through a CRC of
# their bytes instead of the values themselves
import zlib
outs = {k: (np.array([zlib.crc32(v.tobytes())]) if v.size > (1 << 22) else v) for k, v in outs.items()}
np.savez(sys.argv[1], **outs)
print("done", len(outs))
"""


def _run(tile, path, cases=CASES, dtype="bfloat16"):
    env = dict(os.environ, QUTAI_AMD_SPLITK="1")
    env.pop("QUTAI_AMD_GEMM_TILE", None)
    if tile:
        env["QUTAI_AMD_GEMM_TILE"] = tile
    print(f"tile {tile or 'default'} {dtype}", flush=True)
    out = subprocess.run([sys.executable, "-c", CHILD, str(path), str(ROOT), repr(cases), dtype], env=env,
                         capture_output=True, text=True, timeout=110)
    assert out.returncode == 0 and "done" in out.stdout, out.stderr[-2000:]
    return np.load(path)


def test_forced_tiles_are_bit_identical(tmp_path):
    base = _run("L8D2", tmp_path / "L8D2.npz")
    for m, k, n, batch in CASES:
        a, b = normal(10 + m, batch * m * k), normal(20 + n, batch * k * n)
        sa, sb = stored(a, "bfloat16"), stored(b, "bfloat16")
        for ta in (False, True):
            for tb in (False, True):
                exact = np.concatenate([ora.gemm_f64(sa[i * m * k:(i + 1) * m * k], sb[i * k * n:(i + 1) * k * n],
                                                     m, k, n, transpose_left=ta, transpose_right=tb).ravel()
                                        for i in range(batch)])
                got = base[f"{m}_{k}_{n}_{batch}_{ta:d}{tb:d}_float32"]
                assert ora.rel_frobenius(got, exact) <= 1e-2, (m, k, n, batch, ta, tb)
    for tile in ("T", "U", "H", "S", "S2", "N", "W", "R", "P"):
        other = _run(tile, tmp_path / f"{tile}.npz")
        for key in base.files:
            assert np.array_equal(base[key], other[key]), (tile, key)


def test_forced_fp32_tiles_are_bit_identical(tmp_path):
    """fp32 storage: every tile chains v_mfma_f32_32x32x2_f32 over k from 0,
    so forcing any of them (the thin 256x64 tile with its streamed A copies
    included) gives the same bits; the 256x256 result is checked against the
    float64 oracle at the fp32 bar (1e-5)."""
    cases = [(200, 130, 70, 3), (129, 40, 257, 1), (320, 64, 1040, 2), (129, 24, 144, 2), (64, 8, 600, 1)]
    base = _run("L8D2", tmp_path / "L8D2_f32.npz", cases, "float32")
    for m, k, n, batch in cases:
        a, b = normal(10 + m, batch * m * k), normal(20 + n, batch * k * n)
        for ta in (False, True):
            for tb in (False, True):
                exact = np.concatenate([ora.gemm_f64(a[i * m * k:(i + 1) * m * k], b[i * k * n:(i + 1) * k * n],
                                                     m, k, n, transpose_left=ta, transpose_right=tb).ravel()
                                        for i in range(batch)])
                got = base[f"{m}_{k}_{n}_{batch}_{ta:d}{tb:d}_float32"]
                assert ora.rel_frobenius(got, exact) <= 1e-5, (m, k, n, batch, ta, tb)
    for tile in ("H", "S", "S2", "N", "W"):
        other = _run(tile, tmp_path / f"{tile}_f32.npz", cases, "float32")
        for key in base.files:
            assert np.array_equal(base[key], other[key]), (tile, key)


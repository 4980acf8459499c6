"""The amd backend modules export every backend function that the
reference's own callers on the GEMM path invoke, so those callers can run
on ``device="amd"`` once the device is registered (no GPU needed: names and
signatures only)."""
import inspect
import re
from pathlib import Path

import pytest

from qutai_amd.backends import amd, amd_lm

# backend.<name> / get_backend(...).<name> calls of the reference modules on
# the path, with the lines they come from (src/qutai/...)
GENERIC = {
    "core/operations/linalg.py:22,39-55": ["matmul", "gemm", "transpose", "unbroadcast"],
    "core/operations/elementwise.py:10-100": ["broadcast", "add", "subtract", "multiply", "divide", "divide_scalar",
                                              "negate", "unbroadcast", "scale", "exp", "relu_backward",
                                              "gelu_backward", "tanh_backward", "atan_backward"],
    "core/operations/normalization.py:9-25": ["softmax", "multiply", "sum", "broadcast", "subtract"],
    "core/operations/reductions.py:9-35": ["sum", "mean", "broadcast", "scale"],
    "core/operations/transforms.py:10-123": ["transpose", "gather", "gather_slice", "scatter", "scatter_slice",
                                             "concatenate"],
    "core/tensor.py:16-216": ["storage", "full", "add", "copy_into"],
    "core/grad.py:34-65": ["add"],
    "backends/device.py:27-47": ["from_storage", "synchronize", "is_available"],
    "nn/cache.py:5-11": ["concatenate"],
    "lm/layers.py:156-278,436": ["concatenate", "full", "scale"],
    "lm/decoder.py:126": ["full"],
}
# lm backend (`backend(x).<name>`, src/qutai/lm/layers.py:9-17) calls of lm/layers.py, lm/decoder.py
LM = ["add_into", "attention", "attention_backward", "combine", "combine_backward", "embedding",
      "embedding_backward", "gemm", "head_gradient", "head_loss", "head_rows", "head_rows_backward",
      "normal", "prepare_labels", "rms_norm", "rms_norm_backward", "rope", "route_gather", "route_gather_backward",
      "routing", "routing_backward", "silu", "silu_backward", "take"]
# direct module calls `cuda.<name>` / `cuda_lm.<name>` of those callers
DIRECT = {"nn/layers.py:87-88": ["normal", "full", "relu_backward"]}
DIRECT_LM = {"core/operations/transforms.py:19,44": ["embedding", "embedding_backward"]}
# generic functions of those files that are off the contraction path: batch
# and layer normalisation and argmax (classification / sampling)
OFF_PATH = {"batch_norm2d", "batch_norm2d_backward", "channel_stats", "layer_norm", "layer_norm_backward", "argmax",
            "batch_norm"}

# the reference signatures (src/qutai/backends/cuda.py) the callers rely on
SIGNATURES = {
    "broadcast": ["values", "shape", "target"],
    "transpose": ["values", "shape", "axes"],
    "sum": ["values", "shape", "axis"],
    "mean": ["values", "shape", "axis"],
    "unbroadcast": ["values", "shape", "target"],
    "softmax": ["values", "shape", "axis"],
    "divide_scalar": ["values", "value"],
    "concatenate": ["values", "shapes", "axis"],
    "gather": ["values", "positions"],
    "scatter": ["values", "positions", "size"],
    "gather_slice": ["values", "shape", "steps", "offset"],
    "scatter_slice": ["values", "shape", "steps", "offset", "size"],
    "add_into": ["target", "source"],
    "matmul": ["left", "right", "left_shape", "right_shape"],
}


@pytest.mark.parametrize("where", sorted(GENERIC))
def test_generic_functions_exported(where):
    missing = [name for name in GENERIC[where] if not callable(getattr(amd, name, None))]
    assert not missing, f"{where}: amd lacks {missing}"


def test_direct_module_calls_exported():
    for where, names in DIRECT.items():
        assert all(callable(getattr(amd, n, None)) for n in names), where
    for where, names in DIRECT_LM.items():
        assert all(callable(getattr(amd_lm, n, None)) for n in names), where
    # the storage class the serialization / checkpoint code constructs
    assert amd.storage_class is amd.AMDStorage


def test_lm_functions_exported():
    missing = [name for name in LM if not callable(getattr(amd_lm, name, None))]
    assert not missing, missing


@pytest.mark.parametrize("name", sorted(SIGNATURES))
def test_reference_signatures(name):
    parameters = list(inspect.signature(getattr(amd, name)).parameters)
    assert parameters[:len(SIGNATURES[name])] == SIGNATURES[name]


REFERENCE = Path("/root/reference/src/qutai")


@pytest.mark.skipif(not REFERENCE.exists(), reason="the reference source is not on this machine")
def test_lists_cover_the_reference_callers():
    """Re-derive the names from the reference text (read, never imported)."""
    pattern = re.compile(r"\b(?:backend|base|get_backend\([^()]*\))\.([a-z_]+)\(")
    found = set()
    for where in GENERIC:
        text = (REFERENCE / where.split(":")[0]).read_text(encoding="utf8")
        found |= set(pattern.findall(text))
    lm_text = "".join((REFERENCE / f).read_text(encoding="utf8") for f in ("lm/layers.py", "lm/decoder.py"))
    lm_found = set(re.findall(r"\bb\.([a-z_]+)\(", lm_text)) | set(re.findall(r"backend\([^()]*\)\.([a-z_]+)\(",
                                                                               lm_text))
    listed = {name for names in GENERIC.values() for name in names}
    assert found - OFF_PATH <= listed, sorted(found - OFF_PATH - listed)
    for table, module in ((DIRECT, "cuda"), (DIRECT_LM, "cuda_lm")):
        for where, names in table.items():
            text = (REFERENCE / where.split(":")[0]).read_text(encoding="utf8")
            assert set(re.findall(rf"\b{module}\.([a-z_]+)\(", text)) <= set(names), where
    assert lm_found <= set(LM) | listed, sorted(lm_found - set(LM) - listed)

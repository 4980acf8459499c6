"""Mixed-precision switch of the LM layers (src/qutai/lm/precision.py:6-11):
inside ``autocast()`` fp32 weights meet bf16 activations on the bf16 MFMA
path; parameters and their gradients stay fp32."""
from __future__ import annotations

from contextlib import contextmanager

from ..backends.precision import set_matmul_precision


@contextmanager
def autocast(enabled: bool = True, *, dtype: str = "bfloat16"):
    if dtype != "bfloat16":
        raise ValueError("autocast supports bfloat16 only")
    with set_matmul_precision(dtype if enabled else None):
        yield

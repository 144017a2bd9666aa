"""Global precision switches, with the reference's names (src/fdwt/config.py:17-18), and the
rule that turns them into a precision mode (src/fdwt/kernels/conv.py:332-338).

``resolve_precision(dtype)`` returns the mode for inputs of ``dtype`` (the caller's dtype,
before any upcast):

* ``"ieee"``: full fp32 arithmetic (fp64 for fp64 inputs, whatever the switches say);
* ``"bf16"``: bf16 operands with fp32 accumulation, for bf16 / fp16 inputs or when
  ``allow_bf16`` is set;
* ``"tf32"``: when only ``allow_tf32`` is set.  CDNA4 has no TF32 matrix format, so on
  MI355X this mode runs the fp32 kernels: results are those of ``"ieee"``.

Elementwise work, softmax statistics, accumulations and outputs stay fp32 in every mode.
"""

import torch

allow_tf32: bool = False
allow_bf16: bool = False


def resolve_precision(dtype, compute_dtype=None) -> str:
    """Precision mode for inputs of ``dtype`` under the current switches."""
    if (compute_dtype or dtype) == torch.float64:
        return "ieee"
    if dtype in (torch.bfloat16, torch.float16) or allow_bf16:
        return "bf16"
    return "tf32" if allow_tf32 else "ieee"

"""Global precision switches, with the reference's names (src/fdwt/config.py:17-18).

Every kernel of this package computes in full fp32 (plain FMAs) for fp32 / fp16 / bf16
inputs and in fp64 for fp64 inputs, whatever these flags say: the MI355X kernels are
VALU/HBM-bound FIR filters with no reduced-precision matrix path.  The flags are kept so
that code written for the reference runs unchanged; ``resolve_precision`` reports the mode
the reference would pick, for inspection.
"""

allow_tf32: bool = False
allow_bf16: bool = False

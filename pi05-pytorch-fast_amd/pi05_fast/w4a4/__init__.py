"""W4A4 (INT4 weight x INT4 activation, Hadamard-rotated) linear layers for MI355X.

Same public names as the reference package ``pi05_fast.w4a4`` (its ``__init__.py:1-11``).
"""

from pi05_fast.w4a4.apply import apply_w4a4_from_dir, maybe_apply_w4a4_from_env
from pi05_fast.w4a4.linear import W4A4Linear
from pi05_fast.w4a4.pack import int4_gemm_ref, pack_linear_weight

__all__ = [
    "W4A4Linear",
    "apply_w4a4_from_dir",
    "maybe_apply_w4a4_from_env",
    "int4_gemm_ref",
    "pack_linear_weight",
]

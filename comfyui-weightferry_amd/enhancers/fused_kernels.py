"""Codes of the operation the int8 row quantiser may apply before its rotation (the reference's
enhancers/fused_kernels.py:14-18): wf_quant_rows_i8_pre takes them (PRE_NONE inputs also go through
wf_quant_rows_i8)."""
PRE_NONE = 0   # none: the input as it is
PRE_GELU = 1   # GELU of the bf16 input
PRE_MOD = 2    # the scale-and-shift bf16(bf16(x * (1 + scale)) + shift)
PRE_LNMOD = 3  # LayerNorm (no affine), then the scale-and-shift

QUANT_MODES = {"plain": 0, "convrot": 1}

"""Numerical gates shared by the GPU parity tests and the CPU tests that
check those gates can see a composition mistake.

LOGIT_TOL: policy / value / moves-left logits and the decoded value, bf16
kernels against the fp32 reference (2e-2 absolute, the stated tolerance).
TRUNK_MEAN: the trunk output after ln_final (std ~1), bf16 against fp32:
mean absolute error over the summary tokens, and over the live cells.
TRUNK_ROW_REL: the same, per sequence row: |err row| / |reference row| (L2
norms over the channels), largest over the live rows. An error confined to
a few rows (a wrong pad convention, a wrong neighbour) shows here.
F32_RTOL: the fp32 serve mode against the fp32 reference, relative to the
largest magnitude of the compared output (1e-4 relative).
"""

LOGIT_TOL = 2e-2
TRUNK_MEAN = 1e-2
TRUNK_ROW_REL = 4e-2
F32_RTOL = 1e-4

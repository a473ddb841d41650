"""Switches that reproduce reference quirks bit-for-bit instead of fixing them.

``REFERENCE_ROW_CAP``: the reference launches the rows of ``rmsnorm``,
``meanvarnorm`` and ``meanvarnormdx`` on ``workgroup_id.y`` capped at 65 535
with no row loop (reference src/wxx/shaders/layers/rmsnorm.wgsl:23-24,
meanvarnorm.wgsl:28-29, meanvarnormdx.wgsl:27-28;
src/wxx/functional/normalization.py:64,129,347), so every row from 65 535 on
is left as zeros.  Off (the default) computes every row; on, those rows are
written as zeros like the reference's fresh buffers.
"""

REFERENCE_ROW_CAP = False
ROW_CAP = 65535


def row_cap():
    return ROW_CAP if REFERENCE_ROW_CAP else 0

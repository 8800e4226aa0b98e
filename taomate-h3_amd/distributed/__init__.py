"""Linear layers and the quantized-linear dispatch (mirror of taomate_h3.distributed.linear)."""

from .linear import (  # noqa: F401
    ColumnParallelLinear,
    MergedColumnParallelLinear,
    ParallelContext,
    RowParallelLinear,
)

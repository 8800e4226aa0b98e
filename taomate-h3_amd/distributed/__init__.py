"""The quantized-linear dispatch of the parallel linear layers (mirror of taomate_h3.distributed.linear)."""

from .linear import (  # noqa: F401
    _linear,
    _module_fp8_input_scale,
    _module_linear,
    suspend_fp8_activation_calibration,
    use_fp8_activation_scale_policy,
)

"""taomate_h3_amd: MI355X (gfx950) native quantized-linear path for TaoMate-H3.

Host-side mirror of the reference's quantized-linear interface over the C ABI
of ``libtaomate_h3_amd.so`` (include/taomate_h3_amd.h):

* ``ops``                     tensor-level wrappers of the native entry points
* ``inference.w8a8``          H3/inference/w8a8.py (int8 W8A8: policy, streamed
                              weight quantization, workspace, linear)
* ``inference.fused_kernels`` FL/inference/fused_kernels.py:771-820 (FP8 quantizers)
* ``inference.fp8``           FL/inference/fp8.py (FP8 policies and linears) plus
                              per-token x per-channel FP8 W8A8
* ``inference.lora``          H3/inference/lora_checkpoint.py:172-205,261-303
                              (LoRA side branch, fused into the GEMM epilogue)
* ``distributed.linear``      H3/distributed/linear.py:15-191 and
                              FL/distributed/linear.py:50-128 (dispatch + linears)

The directory name is not an identifier; ``__graft_entry__.load_package()``
registers it under the import name ``taomate_h3_amd``.
"""

from __future__ import annotations

__version__ = "0.1.0"

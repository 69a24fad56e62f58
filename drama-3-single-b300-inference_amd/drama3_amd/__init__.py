"""MI355X-native packed FP8 top-8 MoE step with the operator interface of
david6666666/drama-3-single-b300-inference (``src/drama3``).

Modules mirror the reference's: ``kernels`` (route, small_batch_moe,
native_moe, routed_moe, combine_experts*, add_norm, silu_mul), ``moe_input``
(prepare_moe_input, quantize_groups), ``moe_atomic`` (atomic_down),
``packed_prefill`` (PackedLayout, row_metadata), ``runtime_state``
(DeviceRequests).  The decode step over persistent slots is
``pipeline.DecodeStep``, the mixed decode + prefill step ``mixed.MixedStep``
and one whole MoE layer ``moe_layer.MoELayer``.  All compute runs in the HIP
library ``_lib/libdrama3_moe.so``; there is no CPU fallback.
"""

from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent

__all__ = ["PACKAGE_DIR"]

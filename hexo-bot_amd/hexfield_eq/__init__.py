"""MI355X kernels for the hexfield_eq serve ops that run on the 32-slot ray
gather index (``packages/hexfield_eq/python/hexfield_eq/_triton_ray.py``,
``_triton_conv.py``, ``_raytap.py``): ``ray_attn``, ``hex_conv_ln_raytap``
and ``ray_gather_index``, registered as ``torch.ops.hexfield_eq.*``."""

from .ops import (  # noqa: F401
    RAY_GATHER_SLOTS,
    RAY_REACH,
    RAYLEN_SLOTS,
    build_ray_gather_index,
    build_tap_reach,
    hex_conv_ln_raytap,
    launch_conv_ln_raytap,
    launch_ray_attn,
    pack_raytap_weight,
    ray_attn,
    slot_offset_table,
    tap_axis_dir,
    tap_ray_slot_lut,
    tap_raylen_slots,
)

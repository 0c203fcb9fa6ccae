"""shrimp — the Shrimp network's serve forward, built for MI355X (gfx950).

Same public surface as the reference package (constants, geometry, support,
features; model.ShrimpNet; inference.ShrimpEvaluator; the shrimp::* ops);
the forward runs on hand-written HIP kernels behind the C ABI in
``include/shrimp_hip.h``.
"""

from . import constants, features, geometry, support

__all__ = ["constants", "geometry", "support", "features"]

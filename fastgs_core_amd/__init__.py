"""fastgs_core_amd -- MI355X-native FastGS differentiable rasterizer.

Drop-in for the reference package ``fastgs_core`` (a1091150/fastgs_core,
python_package/fastgs_core/__init__.py re-exports ``_fastgs_core``): the
same functions, signatures, dict keys and autograd routes, computed by the
hand-written HIP kernels in ``libfastgs_hip.so``.
"""
from .densify import (  # noqa: F401
    DensifyConfig,
    FastGSTrainLoop,
    GaussianTrainState,
    LoopConfig,
    OptimConfig,
    compute_scene_extent,
)
from .loss import l1_loss, l1_ssim_loss, mse_loss  # noqa: F401
from .train import (  # noqa: F401
    FastGSOptimizerPolicy,
    FusedAdam,
    OptimizerPolicyConfig,
    activate,
    expon_lr_func,
)
from .rasterizer import (  # noqa: F401
    WaitError,
    binning_forward,
    dummy_add,
    dummy_array_size,
    preprocess_forward,
    rasterize_forward,
    rasterize_gaussians,
    rasterize_gaussians_forward,
    tile_prep_forward,
)

__all__ = [
    "rasterize_gaussians",
    "rasterize_gaussians_forward",
    "preprocess_forward",
    "binning_forward",
    "tile_prep_forward",
    "rasterize_forward",
    "dummy_add",
    "dummy_array_size",
]

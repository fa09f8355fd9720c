"""tops.modules on MI355X: the GLA layer's neighbours of the op (tops/modules/*.py) as
torch modules over HIP kernels."""
from .convolution import ShortConvolution, short_conv, short_conv_step
from .fused_norm_gate import FusedRMSNormGated
from .layernorm import RMSNorm, rms_norm_gated

__all__ = ["RMSNorm", "FusedRMSNormGated", "ShortConvolution", "rms_norm_gated", "short_conv",
           "short_conv_step"]

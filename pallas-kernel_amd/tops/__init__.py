"""tops-hip: MI355X-native (gfx950) gated-linear-attention hot path.

Drop-in for the `tops.ops.gla`, `tops.ops.simple_gla` and `tops.ops.kda`
operators of Fred33146/pallas-kernel: same names, signatures, argument
meaning and assertions, computing through hand-written HIP kernels
(libtops_hip.so) on PyTorch-ROCm device tensors.
"""
__version__ = "0.1.0"

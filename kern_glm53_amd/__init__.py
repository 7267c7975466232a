"""kern_glm53_amd: MI355X (gfx950) kernels for kern-glm53's `glm_deepgemm` matmul path.

The product is `libkg.so` (C ABI: include/kg.h), hand-written HIP for CDNA4; `ops` wraps it for PyTorch-ROCm
device tensors with the reference's op signatures, `synth` generates the benchmark's synthetic operands.
"""
from . import ops  # noqa: F401

__version__ = "0.1.0"

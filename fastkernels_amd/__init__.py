"""fastkernels_amd: MI355X-native (gfx950) kernels for the Qwen3.6 MoE decode
layer and the Gated DeltaNet decode step that feeds it.

Operator API: `fastkernels_amd.kernels.hip` (drop-in for the reference's
`fastkernels.kernels.triton` entry points).  C ABI: include/fastkernels_hip.h.
"""

from .spec import Qwen36A3BSpec, qwen36_35b_a3b_spec, synthetic_qwen36_spec

__version__ = "0.1.0"

__all__ = ["Qwen36A3BSpec", "qwen36_35b_a3b_spec", "synthetic_qwen36_spec", "__version__"]

"""MI355X-native LoRA merge for quantized weights (piper-offload's merge hot path).

Host layer over the gfx950 HIP kernels in ``libpiper_lora_merge.so``:

* ``merge_lora`` / ``LoRA`` / ``LoRATransform`` / ``derive_seed`` -- the
  reference's merge API (P/merge.py, P/lora.py, P/seeding.py);
* the tensor adapters and registry (P/tensor_adapters.py,
  P/tensor_adapter_registry.py) for INT8, scaled FP8, NVFP4, MX, GGUF and
  plain tensors;
* ``kernels`` -- drop-in replacements for the Triton merge functions;
* ``stack`` -- grouped multi-target merges;
* ``routed`` -- routed LoRA: the residual hook (P/lora.py:792-930).
"""

from .adapters import Float8Adapter, GgufAdapter, Int8Adapter, MxAdapter, Nvfp4Adapter, RegularAdapter
from .formats import Float8Weight, GGUFWeight, Int8Weight, MXWeight, NVFP4Weight
from .lora import LoRA, LoRAFactor, LoRATransform, ScaledLoRAFactor
from .merge import merge_lora
from .registry import param_representation, register_adapter, select_adapter
from .routed import install_routed_residual_hook, routed_residual
from .seeding import derive_seed

__version__ = "0.1.0"

__all__ = [
    "Float8Adapter",
    "Float8Weight",
    "GGUFWeight",
    "GgufAdapter",
    "Int8Adapter",
    "Int8Weight",
    "LoRA",
    "LoRAFactor",
    "LoRATransform",
    "MXWeight",
    "MxAdapter",
    "NVFP4Weight",
    "Nvfp4Adapter",
    "RegularAdapter",
    "ScaledLoRAFactor",
    "derive_seed",
    "install_routed_residual_hook",
    "merge_lora",
    "param_representation",
    "register_adapter",
    "routed_residual",
    "select_adapter",
]

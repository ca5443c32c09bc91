"""experts4bit_qlora_amd -- the frozen-expert MoE forward of experts4bit-qlora, MI355X-native.

A drop-in for the path ``enable_fast(model)`` routes ``ExpertsNbit`` / ``Experts4bit`` modules
through: the same module classes, state_dict contract and ``enable_fast`` / ``disable_fast`` /
``fast_available`` entry points, with the arithmetic in hand-written gfx950 HIP kernels behind
a C ABI (``include/e4b_amd.h``, ``libe4b_amd.so``)::

    import experts4bit_qlora_amd as e4b
    experts = e4b.Experts4bit.from_float(gate_up, down, compute_dtype=torch.bfloat16)
    assert e4b.enable_fast(model) > 0
"""
from .experts import Experts4bit, ExpertsNbit, normalize_quant_type
from .fast import disable_fast, enable_fast, fast_available
from .formats.mxfp4 import dequantize_mxfp4
from .lora import ExpertsLoRA
from .arch.deepseek_v4 import DeepseekV4Experts4bit, DeepseekV4ExpertsNbit
from .arch.gptoss import GptOssExperts4bit, GptOssExpertsMxfp4, GptOssExpertsNbit
from .ops import gemm_4bit_grouped, gemm_mxfp4_grouped
from .train import disable_fast_train, enable_fast_train

__version__ = "0.1.0"

__all__ = [
    "Experts4bit",
    "ExpertsNbit",
    "ExpertsLoRA",
    "DeepseekV4Experts4bit",
    "DeepseekV4ExpertsNbit",
    "GptOssExperts4bit",
    "GptOssExpertsNbit",
    "GptOssExpertsMxfp4",
    "dequantize_mxfp4",
    "disable_fast",
    "disable_fast_train",
    "enable_fast",
    "enable_fast_train",
    "fast_available",
    "gemm_4bit_grouped",
    "gemm_mxfp4_grouped",
    "normalize_quant_type",
]

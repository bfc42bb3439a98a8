"""Drop-in for the reference's model module.

``main.py`` loads the model module by name (``importlib.import_module(
"qwen_with_nki")``, main.py:904-908) and uses its
``NeuronQwen3MoeForCausalLM`` class surface (main.py:372-433).  This module
exposes the same names, backed by the MI355X implementation in :mod:`qmoe`.
Importing it has no side effects (no downloads, no device work).
"""

from qmoe.attention import Attention as NeuronQwen3MoEAttention  # noqa: F401
from qmoe.model import (  # noqa: F401
    CausalLMOutput,
    HuggingFaceGenerationAdapter,
    MoENeuronConfig,
    NeuronQwen3MoeDecoderLayer,
    NeuronQwen3MoeForCausalLM,
    NeuronQwen3MoeModel,
    Qwen3MoeInferenceConfig,
    convert_qwen3_moe_hf_to_neuron_state_dict,
    load_pretrained_config,
)
from qmoe.moe import ExpertMLPs as ExpertMLPsV2  # noqa: F401
from qmoe.moe import MoEBlock  # noqa: F401

__all__ = [
    "NeuronQwen3MoeForCausalLM",
    "NeuronQwen3MoeModel",
    "NeuronQwen3MoeDecoderLayer",
    "NeuronQwen3MoEAttention",
    "Qwen3MoeInferenceConfig",
    "MoENeuronConfig",
    "HuggingFaceGenerationAdapter",
    "convert_qwen3_moe_hf_to_neuron_state_dict",
    "load_pretrained_config",
    "ExpertMLPsV2",
    "MoEBlock",
]

"""MI355X (gfx950) decode hot path of the Qwen3.5-2B-shaped hybrid decoder.

Python mirror of the reference engine's kernel / layer / model surface over the C ABI of
libq35.so (include/q35.h).  Import with qwen-3.5_amd/ on sys.path: `import q35`.
"""
from . import _lib
from ._lib import Q35_KN, Q35_KN_TILED, Q35_LAUNCH_GRAPH, Q35_LAUNCH_PERSISTENT, Q35_LAUNCH_STREAM, Q35_NK, Q35Error, dims_2b, make_dims, lib
from .kernels import (Q8FTensor, argmax, gate_proj, q8_embedding_lookup, q8_gemv, q8_gemv_partial_sum, q8_lm_head,
                      release_workspaces, workspace)
from .model import (BatchDecoder, TextForCausalLM, quantize_q8f, safetensors_tensor, synth_model_tensor, synth_normal,
                    synth_uniform)
from .modules import (MLP, Attention, GatedDeltaNet, attention_core_decode, gated_delta_rule_decode,
                      rope_tables)
from .prefill import attention_core_prefill, gate_proj_prompt, gated_delta_rule_prefill, q8_gemm

__all__ = ["Q35_KN", "Q35_KN_TILED", "Q35_NK", "Q35_LAUNCH_STREAM", "Q35_LAUNCH_GRAPH", "Q35_LAUNCH_PERSISTENT", "Q35Error", "dims_2b", "make_dims", "lib", "Q8FTensor", "argmax", "gate_proj",
           "q8_embedding_lookup", "q8_gemv", "q8_gemv_partial_sum", "q8_lm_head", "release_workspaces", "workspace", "TextForCausalLM", "BatchDecoder",
           "quantize_q8f", "safetensors_tensor", "synth_model_tensor", "synth_normal", "synth_uniform", "MLP", "Attention", "GatedDeltaNet",
           "rope_tables", "attention_core_decode", "gated_delta_rule_decode", "attention_core_prefill", "gate_proj_prompt",
           "gated_delta_rule_prefill", "q8_gemm", "_lib"]

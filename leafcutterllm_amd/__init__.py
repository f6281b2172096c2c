"""MI355X-native (gfx950) MoE feed-forward layer behind a C ABI.

The compute lives in liblcmoe.so (HIP kernels + C ABI, include/lcmoe.h); this
package binds it with ctypes and carries the benchmark layer shapes.
"""
from ._lib import (ACT_F16, ACT_F16X2, ROUTE_SIGMOID_GROUP, ROUTE_SOFTMAX, ROUTE_SOFTMAX_RENORM, TYPE_F32,
                   TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, Desc, LcmoeError, Weights, lib)
from .configs import CONFIGS, MODEL_CONFIGS, LayerConfig, ModelConfig, synth_layer, synth_model, synth_x
from .gguf import GgufFile
from .model import Model, ModelDesc
from .moe import (MoeFfn, debug_dequant, debug_rmsnorm, debug_sigmoid, dequantize, matmul,
                  read_bandwidth, sanitize_blocks, shard_matmul)

__all__ = [
    "CONFIGS", "MODEL_CONFIGS", "LayerConfig", "ModelConfig", "synth_layer", "synth_model",
    "synth_x", "MoeFfn", "Model", "ModelDesc", "GgufFile", "Desc", "Weights",
    "LcmoeError", "lib", "dequantize", "sanitize_blocks", "debug_dequant", "debug_rmsnorm", "debug_sigmoid", "shard_matmul", "matmul", "read_bandwidth", "TYPE_F32", "TYPE_Q4_0", "TYPE_Q8_0",
    "TYPE_Q4_K", "TYPE_Q6_K", "ACT_F16", "ACT_F16X2", "ROUTE_SOFTMAX_RENORM", "ROUTE_SOFTMAX", "ROUTE_SIGMOID_GROUP",
]

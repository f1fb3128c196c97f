"""llapis_amd -- MI355X-native dual-precision MoE expert FFN (router softmax/top-k,
gate_up -> GeGLU -> down over hot Q4_K/Q5_0 and cold IQ2_S/IQ4_NL experts),
behind the reference's moert island ABI and ggml_moe_dual operator."""
from ._lib import (ACT_CPU, ACT_Q8_1, F32, GELU_TABLE, GELU_TANH, IQ2_S, IQ4_NL, Q4_K, Q5_0, Q8_0, Q8_1, Q8_K,
                   SLOT_FILLING, SLOT_FREE, SLOT_READY, LlapisError, lib)
from .moe import (DeviceLayer, DualLayer, LayerSpec, Residency, combine, geglu, make_layer, quantize, residual_rmsnorm,
                  row_size,
                  seed_for, synth_normal, tune_router_bias, zipf_hot_set)

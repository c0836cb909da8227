"""vallmo.jl_amd — the gated full-attention path of Vallmo.jl on MI355X (gfx950).

Hand-written CDNA4 HIP kernels in ``csrc/`` built into ``libvallmo_attn.so``
(C ABI: include/vallmo_attn.h); this package is the host-side mirror of the
reference's operator and layer call surface (src/kernels/*.jl,
src/llm/qwen35.jl, src/llm/generate.jl) over that ABI.

The directory name is not a Python identifier; load it with
``__graft_entry__.load_package()`` (registered as module ``vallmo_amd``).
"""
from ._lib import (ArgumentError, BoundsError, DimensionMismatch, HIPError,  # noqa: F401
                   UnsupportedShape,
                   LIB_PATH, EXPORTED)
from .sizes import sizes  # noqa: F401
from .ops import (attention, attention_, decode_attention, decode_attention_,  # noqa: F401
                  decode_scratch_bytes, embed_, fill_normal_, fused_add_rms_norm,
                  fused_add_rms_norm_, knorm_rope_append_, linear, linear_,
                  linear_tune, linear_workspace_bytes, lm_head_argmax, lm_head_argmax_,
                  lm_head_argmax_scratch_bytes, qnorm_rope_, rms_norm, rms_norm_, rope_tables,
                  sigmoid, sigmoid_gate_, silu_mul_, causal_conv1d, causal_conv1d_,
                  causal_conv1d_sequence, causal_conv1d_sequence_, fused_deltanet_decode,
                  fused_deltanet_decode_, deltanet_recurrent_decode, deltanet_recurrent_decode_,
                  deltanet_sequence, deltanet_sequence_, deltanet_prefill_prep_,
                  deltanet_conv_prep_, gated_rms_norm_,
                  linear_add_rms_norm_, linear_add_rms_norm_workspace_bytes,
                  linear_silu_mul_, linear_silu_mul_workspace_bytes,
                  linear_causal_conv1d_, linear_causal_conv1d_workspace_bytes,
                  linear_deltanet_decode_,
                  deltanet_sequence_chunked_, deltanet_sequence_workspace_bytes,
                  deltanet_sequence_chunked_gated_norm_)
from .layer import (AttnConfig, AttnLayer, AttnModel, CaptureSession, Generation,  # noqa: F401
                    StagedV, attn_layer, decode_, forward, gated_attn_decode_, gated_attn_prefill)
from .model import (Model, ModelConfig, generate_, generate_captured_, mlp_,  # noqa: F401
                    prefill_, random_model, step_)
from .deltanet_layer import (DeltaNetConfig, DeltaNetLayer, DeltaNetSpace,  # noqa: F401
                             deltanet_layer)
from . import _lib  # noqa: F401

__version__ = "0.1.0"

"""MI355X-native Gated DeltaNet operator (prefill, its backward, decode) behind the
reference's operator API; see pseudobrain_amd.gated_deltanet. The layer-side
prologue and epilogue around it are in pseudobrain_amd.layer."""
from .gated_deltanet import (  # noqa: F401
    CHUNK, KERNELS, SEQUENTIAL_MAX, chunk_bwd, chunk_decumulate, chunk_fwd, chunk_fwd_slots, chunk_residuals,
    chunk_slots_, delta_rule_hip, delta_rule_sequential, gated_delta_chunk, gated_delta_chunk_backward,
    gated_delta_chunk_fla, gated_delta_chunk_fla_backward, gated_delta_rule, hip_usable, recurrent_fwd,
    recurrent_step_, register_reference_ops, select_kernel,
)
from .layer import decode_layer_step, layer_epilogue, layer_prologue, layer_prologue_varlen  # noqa: F401,E402

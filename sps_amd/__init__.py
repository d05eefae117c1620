"""sps_amd: MI355X-native (gfx950) attention hot path of the SPS Transformer.

Drop-in replacements for the reference's attention entry points:
  prefill / training: ``sps_sliding_attention``, ``reverse_sps_sliding_attention``, ``full_attention``
  decode:             ``KVSegment``, ``triton_segmented_q1_attention``, ``triton_segmented_q2_attention``,
                      ``masked_kv_attention``, ``fused_sps_kv_update`` (KV-cache update),
                      ``segmented_q{1,2}_attention_with_kv_update`` (a decode step's attention and
                      KV update in the attention's launches)
  pre-attention:      ``apply_rotary_emb``, ``rope_qkv_for_attention`` (RoPE + casts + layout, one launch)
  prefill -> decode:  ``prefill_to_decode``, ``materialize_prefill_layer_state`` (decode caches, one launch)
  document ids:       ``document_ids`` (EOS / left-pad rules, interleaved for the SPS families)
All compute runs in libsps_attn.so (hand-written HIP kernels); see include/sps_attn.h.
"""

from .attention import full_attention, reverse_sps_sliding_attention, sps_sliding_attention
from .decode_attention import (
    KVSegment,
    masked_kv_attention,
    triton_segmented_q1_attention,
    triton_segmented_q2_attention,
)
from .decode_attention_fast import (
    fused_sps_kv_update,
    segmented_q1_attention_with_kv_update,
    segmented_q2_attention_with_kv_update,
)
from .doc_ids import document_ids, left_padded_document_ids
from .integration import install_into_modeling
from .rope import apply_rotary_emb, rope_qkv_for_attention
from .prefill_state import materialize_prefill_layer_state, prefill_to_decode

__all__ = [
    "sps_sliding_attention",
    "reverse_sps_sliding_attention",
    "full_attention",
    "KVSegment",
    "triton_segmented_q1_attention",
    "triton_segmented_q2_attention",
    "masked_kv_attention",
    "fused_sps_kv_update",
    "segmented_q1_attention_with_kv_update",
    "segmented_q2_attention_with_kv_update",
    "document_ids",
    "left_padded_document_ids",
    "install_into_modeling",
    "apply_rotary_emb",
    "rope_qkv_for_attention",
    "prefill_to_decode",
    "materialize_prefill_layer_state",
]

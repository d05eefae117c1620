"""Routes the reference modeling code's attention imports to sps_amd.

The reference modeling package (lil-lab/sps, ``src/modeling``) binds its attention kernels by these
module paths and names:

    modeling.models.attention.triton_sps_flash_attention.sps_sliding_attention
        (imported as triton_sps_sliding_attention by sps/core.py:27-32)
    modeling.models.attention.triton_reverse_sps_flash_attention.reverse_sps_sliding_attention
        (imported as triton_reverse_sps_sliding_attention by reverse_sps/core.py:33-38)
    modeling.models.attention.triton_full_flash_attention.full_attention
        (imported as triton_full_attention by full_attention_model.py:44-47)
    modeling.models.utils.decode_attention.{KVSegment, masked_kv_attention,
        triton_segmented_q1_attention, triton_segmented_q2_attention}
        (reverse_sps/inference.py:19-23, full_attention_model.py:41)
    modeling.models.utils.decode_attention_fast.fused_sps_kv_update
        (reverse_sps/inference.py:24)
    ReverseSPSInferenceMixin._materialize_prefill_layer_state
        (reverse_sps/inference.py:568-613; the SPS and delayed-state models inherit it)

``install_into_modeling()`` registers modules under the three attention paths and the KV-update
path whose functions are sps_amd's, and rebinds the names in any of the consumer modules already
imported. Call it before (or after) importing the modeling package; it never imports Triton or the
reference kernels.
"""

from __future__ import annotations

import sys
import types

from . import attention as _attn
from . import decode_attention as _dec
from . import decode_attention_fast as _fast

_ATTENTION_MODULES = {
    "modeling.models.attention.triton_sps_flash_attention": {"sps_sliding_attention": _attn.sps_sliding_attention},
    "modeling.models.attention.triton_reverse_sps_flash_attention": {
        "reverse_sps_sliding_attention": _attn.reverse_sps_sliding_attention
    },
    "modeling.models.attention.triton_full_flash_attention": {"full_attention": _attn.full_attention},
    "modeling.models.utils.decode_attention_fast": {"fused_sps_kv_update": _fast.fused_sps_kv_update},
}

_DECODE_NAMES = {
    "KVSegment": _dec.KVSegment,
    "masked_kv_attention": _dec.masked_kv_attention,
    "triton_segmented_q1_attention": _dec.triton_segmented_q1_attention,
    "triton_segmented_q2_attention": _dec.triton_segmented_q2_attention,
}

# Consumer module -> {bound name: replacement}
_CONSUMERS = {
    "modeling.models.sps.core": {"triton_sps_sliding_attention": _attn.sps_sliding_attention},
    "modeling.models.reverse_sps.core": {"triton_reverse_sps_sliding_attention": _attn.reverse_sps_sliding_attention},
    "modeling.models.full_attention_model": {
        "triton_full_attention": _attn.full_attention,
        "KVSegment": _dec.KVSegment,
        "masked_kv_attention": _dec.masked_kv_attention,
    },
    "modeling.models.reverse_sps.inference": {
        "KVSegment": _dec.KVSegment,
        "masked_kv_attention": _dec.masked_kv_attention,
        "triton_segmented_q2_attention": _dec.triton_segmented_q2_attention,
        "fused_sps_kv_update": _fast.fused_sps_kv_update,
    },
}


def install_into_modeling(rope: bool = False) -> list[str]:
    """Installs the drop-in; returns the module names that were created or patched.

    ``rope=True`` also rebinds ``modeling.models.model.apply_rotary_emb`` (model.py:201-230, called
    by every attention module) to sps_amd's GPU kernel. It is opt-in because the reference also
    runs that function on CPU tensors, which sps_amd does not support."""
    touched = []
    inf = sys.modules.get("modeling.models.reverse_sps.inference")
    mixin = getattr(inf, "ReverseSPSInferenceMixin", None) if inf is not None else None
    if mixin is not None:
        # Only the batched (GPU) prefill path calls it (reverse_sps/inference.py:518-530, 669).
        from .prefill_state import materialize_prefill_layer_state

        mixin._materialize_prefill_layer_state = materialize_prefill_layer_state
        touched.append("modeling.models.reverse_sps.inference.ReverseSPSInferenceMixin")
    if rope:
        from . import rope as _rope

        mod = sys.modules.get("modeling.models.model")
        if mod is not None:
            mod.apply_rotary_emb = _rope.apply_rotary_emb
            touched.append("modeling.models.model")
    for name, attrs in _ATTENTION_MODULES.items():
        mod = sys.modules.get(name)
        if mod is None:
            mod = types.ModuleType(name, f"sps_amd drop-in for {name}")
            sys.modules[name] = mod
        for attr, fn in attrs.items():
            setattr(mod, attr, fn)
        touched.append(name)
    dec = sys.modules.get("modeling.models.utils.decode_attention")
    if dec is not None:
        for attr, obj in _DECODE_NAMES.items():
            setattr(dec, attr, obj)
        touched.append("modeling.models.utils.decode_attention")
    for name, attrs in _CONSUMERS.items():
        mod = sys.modules.get(name)
        if mod is None:
            continue
        for attr, obj in attrs.items():
            setattr(mod, attr, obj)
        touched.append(name)
    return touched

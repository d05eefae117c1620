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
    modeling.models.model.{apply_rotary_emb, generate_left_padded_document_idx}
        (model.py:201-230 and :70-99; imported by name by the attention modules and the models)
    ReverseSPSInferenceMixin._materialize_prefill_layer_state
        (reverse_sps/inference.py:568-613; the SPS and delayed-state models inherit it)

``install_into_modeling()`` registers modules under the three attention paths and the KV-update
path whose functions are sps_amd's, and rebinds the names in any of the consumer modules already
imported. Call it before (or after) importing the modeling package; it never imports Triton or the
reference kernels.

Functions the reference also runs on CPU tensors (``masked_kv_attention``: the padded-SDPA path used
by CPU decoding, decode_attention.py:637-698; ``apply_rotary_emb``; the document-id function) are
rebound to a dispatcher that keeps the module's original function: CUDA tensors go to the HIP kernels,
anything else to the original, so the reference's CPU paths keep working after the install.
"""

from __future__ import annotations

import functools
import sys
import types

from . import attention as _attn
from . import decode_attention as _dec
from . import decode_attention_fast as _fast
from . import doc_ids as _ids
from . import rope as _rope

_ATTENTION_MODULES = {
    "modeling.models.attention.triton_sps_flash_attention": {"sps_sliding_attention": _attn.sps_sliding_attention},
    "modeling.models.attention.triton_reverse_sps_flash_attention": {
        "reverse_sps_sliding_attention": _attn.reverse_sps_sliding_attention
    },
    "modeling.models.attention.triton_full_flash_attention": {"full_attention": _attn.full_attention},
    "modeling.models.utils.decode_attention_fast": {"fused_sps_kv_update": _fast.fused_sps_kv_update},
}

# GPU-only replacements (the reference versions need CUDA too).
_DECODE_NAMES = {
    "KVSegment": _dec.KVSegment,
    "triton_segmented_q1_attention": _dec.triton_segmented_q1_attention,
    "triton_segmented_q2_attention": _dec.triton_segmented_q2_attention,
}

# Name -> (sps_amd GPU function, predicate on the call's arguments: True sends it to the GPU function).
_DEVICE_DISPATCHED = {
    "masked_kv_attention": (_dec.masked_kv_attention,
                            lambda *a, **kw: (kw["q_BxHxD"] if "q_BxHxD" in kw else a[0]).is_cuda),
    "apply_rotary_emb": (_rope.apply_rotary_emb, lambda *a, **kw: (kw["xq"] if "xq" in kw else a[0]).is_cuda),
    "generate_left_padded_document_idx": (
        _ids.left_padded_document_ids, lambda *a, **kw: (kw["idx_BxT"] if "idx_BxT" in kw else a[0]).is_cuda),
}

# Module that defines each dispatched name (where the original lives).
_HOME = {
    "masked_kv_attention": "modeling.models.utils.decode_attention",
    "apply_rotary_emb": "modeling.models.model",
    "generate_left_padded_document_idx": "modeling.models.model",
}

# Consumer module -> names it binds at import time.
# (sps/core.py looks apply_rotary_emb up in modeling.models.model at call time, :50; the others
# import it by name: full_attention_model.py:26-32, reverse_sps/core.py:16-19,
# reverse_sps/inference.py:13-14.)
_CONSUMERS = {
    "modeling.models.sps.core": {"triton_sps_sliding_attention": _attn.sps_sliding_attention},
    "modeling.models.reverse_sps.core": {
        "triton_reverse_sps_sliding_attention": _attn.reverse_sps_sliding_attention,
        "apply_rotary_emb": None,
        "generate_left_padded_document_idx": None,
    },
    "modeling.models.full_attention_model": {
        "triton_full_attention": _attn.full_attention,
        "KVSegment": _dec.KVSegment,
        "masked_kv_attention": None,
        "apply_rotary_emb": None,
        "generate_left_padded_document_idx": None,
    },
    "modeling.models.reverse_sps.inference": {
        "KVSegment": _dec.KVSegment,
        "masked_kv_attention": None,
        "apply_rotary_emb": None,
        "triton_segmented_q2_attention": _dec.triton_segmented_q2_attention,
        "fused_sps_kv_update": _fast.fused_sps_kv_update,
    },
}
# (None: the device dispatcher of that name.)


def _dispatcher(name: str, original):
    """The device dispatcher of `name` around `original` (None: every call goes to the GPU function)."""
    gpu_fn, on_gpu = _DEVICE_DISPATCHED[name]
    original = getattr(original, "__sps_amd_original__", original)

    @functools.wraps(gpu_fn)
    def fn(*args, **kwargs):
        if original is None or on_gpu(*args, **kwargs):
            return gpu_fn(*args, **kwargs)
        return original(*args, **kwargs)

    fn.__sps_amd_original__ = original
    return fn


def install_into_modeling() -> list[str]:
    """Installs the drop-in; returns the module names that were created or patched."""
    touched = []
    inf = sys.modules.get("modeling.models.reverse_sps.inference")
    mixin = getattr(inf, "ReverseSPSInferenceMixin", None) if inf is not None else None
    if mixin is not None:
        # Only the batched (GPU) prefill path calls it (reverse_sps/inference.py:518-530, 669).
        from .prefill_state import materialize_prefill_layer_state

        mixin._materialize_prefill_layer_state = materialize_prefill_layer_state
        touched.append("modeling.models.reverse_sps.inference.ReverseSPSInferenceMixin")
    for name, attrs in _ATTENTION_MODULES.items():
        mod = sys.modules.get(name)
        if mod is None:
            mod = types.ModuleType(name, f"sps_amd drop-in for {name}")
            sys.modules[name] = mod
        for attr, fn in attrs.items():
            setattr(mod, attr, fn)
        touched.append(name)
    # One dispatcher per name, wrapping the original of the module that defines it.
    dispatchers = {}
    for name, home in _HOME.items():
        mod = sys.modules.get(home)
        dispatchers[name] = _dispatcher(name, getattr(mod, name, None) if mod is not None else None)
        if mod is not None:
            setattr(mod, name, dispatchers[name])
            touched.append(f"{home}.{name}")
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
            if obj is None:
                if not hasattr(mod, attr):
                    continue
                obj = dispatchers[attr]
                if dispatchers[attr].__sps_amd_original__ is None:
                    # The defining module is not loaded: keep the consumer's own binding as the original.
                    obj = _dispatcher(attr, getattr(mod, attr))
            setattr(mod, attr, obj)
        touched.append(name)
    return touched

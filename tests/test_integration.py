"""install_into_modeling routes the reference modeling package's names to sps_amd (CPU only: fake
modules stand in for the reference's, which are not imported)."""

import sys
import types

import sps_amd
from sps_amd import decode_attention_fast, prefill_state, rope


def test_install_into_modeling_rebinds_every_entry_point(monkeypatch):
    names = ["modeling.models.sps.core", "modeling.models.reverse_sps.core", "modeling.models.full_attention_model",
             "modeling.models.reverse_sps.inference", "modeling.models.utils.decode_attention",
             "modeling.models.model"]
    mods = {n: types.ModuleType(n) for n in names}

    class ReverseSPSInferenceMixin:
        pass

    mods["modeling.models.reverse_sps.inference"].ReverseSPSInferenceMixin = ReverseSPSInferenceMixin
    for n, m in mods.items():
        monkeypatch.setitem(sys.modules, n, m)
    for n in ["modeling.models.attention.triton_sps_flash_attention",
              "modeling.models.attention.triton_reverse_sps_flash_attention",
              "modeling.models.attention.triton_full_flash_attention",
              "modeling.models.utils.decode_attention_fast"]:
        monkeypatch.delitem(sys.modules, n, raising=False)
    touched = sps_amd.install_into_modeling(rope=True)
    assert sys.modules["modeling.models.attention.triton_sps_flash_attention"].sps_sliding_attention is \
        sps_amd.sps_sliding_attention
    assert sys.modules["modeling.models.utils.decode_attention_fast"].fused_sps_kv_update is \
        decode_attention_fast.fused_sps_kv_update
    assert mods["modeling.models.sps.core"].triton_sps_sliding_attention is sps_amd.sps_sliding_attention
    assert mods["modeling.models.reverse_sps.inference"].fused_sps_kv_update is decode_attention_fast.fused_sps_kv_update
    assert mods["modeling.models.reverse_sps.inference"].triton_segmented_q2_attention is \
        sps_amd.triton_segmented_q2_attention
    assert mods["modeling.models.utils.decode_attention"].masked_kv_attention is sps_amd.masked_kv_attention
    assert mods["modeling.models.model"].apply_rotary_emb is rope.apply_rotary_emb
    assert ReverseSPSInferenceMixin._materialize_prefill_layer_state is prefill_state.materialize_prefill_layer_state
    assert "modeling.models.model" in touched

"""install_into_modeling routes the reference modeling package's names to sps_amd (CPU: stand-in
modules play the reference's, which are not imported)."""

import sys
import types

import pytest
import torch

import sps_amd
from sps_amd import decode_attention_fast, integration, prefill_state

MODULES = ["modeling.models.sps.core", "modeling.models.reverse_sps.core", "modeling.models.full_attention_model",
           "modeling.models.reverse_sps.inference", "modeling.models.utils.decode_attention",
           "modeling.models.model"]


class _CudaLike:
    """Stands in for a CUDA tensor where only the device test of the dispatch looks at it."""

    is_cuda = True


def _install_stand_ins(monkeypatch):
    mods = {n: types.ModuleType(n) for n in MODULES}
    calls = []

    def original(tag):
        def fn(*args, **kwargs):
            calls.append(("original", tag))
            return tag

        return fn

    class ReverseSPSInferenceMixin:
        pass

    mods["modeling.models.reverse_sps.inference"].ReverseSPSInferenceMixin = ReverseSPSInferenceMixin
    mods["modeling.models.utils.decode_attention"].masked_kv_attention = original("masked_kv_attention")
    mods["modeling.models.model"].apply_rotary_emb = original("apply_rotary_emb")
    mods["modeling.models.model"].generate_left_padded_document_idx = original("document_idx")
    # Consumers bound the originals by name when they were imported.
    for consumer in ("modeling.models.full_attention_model", "modeling.models.reverse_sps.inference"):
        mods[consumer].masked_kv_attention = mods["modeling.models.utils.decode_attention"].masked_kv_attention
    for consumer in ("modeling.models.full_attention_model", "modeling.models.reverse_sps.core"):
        mods[consumer].generate_left_padded_document_idx = \
            mods["modeling.models.model"].generate_left_padded_document_idx
    for consumer in ("modeling.models.full_attention_model", "modeling.models.reverse_sps.core",
                     "modeling.models.reverse_sps.inference"):
        mods[consumer].apply_rotary_emb = mods["modeling.models.model"].apply_rotary_emb
    for n, m in mods.items():
        monkeypatch.setitem(sys.modules, n, m)
    for n in ["modeling.models.attention.triton_sps_flash_attention",
              "modeling.models.attention.triton_reverse_sps_flash_attention",
              "modeling.models.attention.triton_full_flash_attention",
              "modeling.models.utils.decode_attention_fast"]:
        monkeypatch.delitem(sys.modules, n, raising=False)
    # Record which GPU function a CUDA call reaches (the real ones need a GPU).
    gpu_calls = []
    patched = {}
    for name, (fn, pred) in integration._DEVICE_DISPATCHED.items():
        def rec(*args, _name=name, **kwargs):
            gpu_calls.append(_name)
            return "gpu"

        patched[name] = (rec, pred)
    monkeypatch.setattr(integration, "_DEVICE_DISPATCHED", patched)
    return mods, calls, gpu_calls, ReverseSPSInferenceMixin


def test_install_into_modeling_rebinds_every_entry_point(monkeypatch):
    mods, _, _, mixin = _install_stand_ins(monkeypatch)
    touched = sps_amd.install_into_modeling()
    assert sys.modules["modeling.models.attention.triton_sps_flash_attention"].sps_sliding_attention is \
        sps_amd.sps_sliding_attention
    assert sys.modules["modeling.models.utils.decode_attention_fast"].fused_sps_kv_update is \
        decode_attention_fast.fused_sps_kv_update
    assert mods["modeling.models.sps.core"].triton_sps_sliding_attention is sps_amd.sps_sliding_attention
    assert mods["modeling.models.reverse_sps.core"].triton_reverse_sps_sliding_attention is \
        sps_amd.reverse_sps_sliding_attention
    assert mods["modeling.models.full_attention_model"].triton_full_attention is sps_amd.full_attention
    assert mods["modeling.models.reverse_sps.inference"].fused_sps_kv_update is decode_attention_fast.fused_sps_kv_update
    assert mods["modeling.models.reverse_sps.inference"].triton_segmented_q2_attention is \
        sps_amd.triton_segmented_q2_attention
    assert mods["modeling.models.utils.decode_attention"].triton_segmented_q1_attention is \
        sps_amd.triton_segmented_q1_attention
    assert mixin._materialize_prefill_layer_state is prefill_state.materialize_prefill_layer_state
    assert "modeling.models.model.apply_rotary_emb" in touched


def test_cpu_calls_keep_the_reference_path_and_cuda_calls_reach_the_kernels(monkeypatch):
    # masked_kv_attention is the reference's only CPU attention (decode_attention.py:637-698, used by
    # CPU forward_efficient and Standard-model CPU decoding): after the install, CPU tensors still
    # reach it, CUDA tensors reach the HIP path. Likewise apply_rotary_emb and the document ids.
    mods, calls, gpu_calls, _ = _install_stand_ins(monkeypatch)
    sps_amd.install_into_modeling()
    cpu = torch.zeros(2, 3, 4)
    for consumer in ("modeling.models.utils.decode_attention", "modeling.models.full_attention_model",
                     "modeling.models.reverse_sps.inference"):
        fn = mods[consumer].masked_kv_attention
        assert fn(cpu, [], attn_dtype=torch.float32) == "masked_kv_attention"
        assert fn(q_BxHxD=cpu, segments=[], attn_dtype=torch.float32) == "masked_kv_attention"
        assert fn(_CudaLike(), [], attn_dtype=torch.bfloat16) == "gpu"
    # apply_rotary_emb: where it is defined, and in the three modules that import it by name
    # (full_attention_model.py:26-32, reverse_sps/core.py:16-19, reverse_sps/inference.py:13-14).
    for consumer in ("modeling.models.model", "modeling.models.full_attention_model",
                     "modeling.models.reverse_sps.core", "modeling.models.reverse_sps.inference"):
        rope = mods[consumer].apply_rotary_emb
        assert rope(cpu, cpu, cpu) == "apply_rotary_emb"
        assert rope(_CudaLike(), None, None) == "gpu"
        assert rope(xq=_CudaLike(), xk=None, freqs_cis=None) == "gpu"
    assert gpu_calls.count("apply_rotary_emb") == 8
    for consumer in ("modeling.models.model", "modeling.models.full_attention_model",
                     "modeling.models.reverse_sps.core"):
        ids = mods[consumer].generate_left_padded_document_idx
        assert ids(cpu, eos_token_id=1, pad_token_id=0) == "document_idx"
        assert ids(_CudaLike(), eos_token_id=1, pad_token_id=0) == "gpu"
    assert ("original", "masked_kv_attention") in calls and "masked_kv_attention" in gpu_calls
    assert gpu_calls.count("generate_left_padded_document_idx") == 3


def test_second_install_does_not_stack_dispatchers(monkeypatch):
    mods, calls, gpu_calls, _ = _install_stand_ins(monkeypatch)
    sps_amd.install_into_modeling()
    first = mods["modeling.models.utils.decode_attention"].masked_kv_attention
    sps_amd.install_into_modeling()
    second = mods["modeling.models.utils.decode_attention"].masked_kv_attention
    assert second.__sps_amd_original__ is first.__sps_amd_original__
    calls.clear()
    assert second(torch.zeros(1, 1, 1), [], attn_dtype=torch.float32) == "masked_kv_attention"
    assert calls == [("original", "masked_kv_attention")]


def test_without_the_modeling_package_gpu_calls_only(monkeypatch):
    for n in MODULES:
        monkeypatch.delitem(sys.modules, n, raising=False)
    for n in ["modeling.models.attention.triton_sps_flash_attention",
              "modeling.models.attention.triton_reverse_sps_flash_attention",
              "modeling.models.attention.triton_full_flash_attention",
              "modeling.models.utils.decode_attention_fast"]:
        monkeypatch.delitem(sys.modules, n, raising=False)
    touched = sps_amd.install_into_modeling()
    assert "modeling.models.attention.triton_full_flash_attention" in touched
    with pytest.raises(RuntimeError, match="GPU only"):
        sps_amd.masked_kv_attention(torch.zeros(1, 1, 64), [], attn_dtype=torch.float32)


def test_fused_decode_wrappers_take_both_reference_signatures():
    # segmented_q{1,2}_attention_with_kv_update take the keyword arguments of the attention call they
    # replace (triton_segmented_q{1,2}_attention) followed by fused_sps_kv_update's, under the same names.
    import inspect

    from sps_amd import decode_attention as DA
    from sps_amd import decode_attention_fast as DF

    upd = [p for p in inspect.signature(DF.fused_sps_kv_update).parameters]
    for fused, attn in ((DF.segmented_q2_attention_with_kv_update, DA.triton_segmented_q2_attention),
                        (DF.segmented_q1_attention_with_kv_update, DA.triton_segmented_q1_attention)):
        got = list(inspect.signature(fused).parameters)
        want = [p for p in inspect.signature(attn).parameters if not p.startswith("_")] + upd
        assert got == want, (fused.__name__, got, want)

"""Host-side behaviour of the drop-in enhancers.gguf_dequant against a stand-in ComfyUI-GGUF (CPU only): install /
uninstall / idempotence and the WEIGHTFERRY_GGUF_TRITON gate (enhancers/gguf_dequant.py:544-576 of the
reference), the None -> ComfyUI-GGUF fallback and the used / fallback counters (:521-541,579-583), the K-quant
gate (:264-274), and the plain-LoRA eligibility rules of lora_factors (:329-355)."""
import pytest
import torch

from conftest import sub


@pytest.fixture
def gd():
    m = sub("enhancers.gguf_dequant")
    m.stats(reset=True)
    yield m
    m._KQUANTS = None
    m.uninstall()


def test_install_patches_and_uninstall_restores(gd, fake_gguf):
    orig_dq, orig_gw = fake_gguf.dequantize_tensor, fake_gguf.GGMLLayer.get_weight
    assert gd.install(force=True) is True
    assert fake_gguf.dequantize_tensor is not orig_dq and fake_gguf.dequantize_tensor._weightferry
    assert fake_gguf.GGMLLayer.get_weight._weightferry
    assert gd.install(force=True) is True                       # idempotent
    patched = fake_gguf.dequantize_tensor
    assert gd.install(force=True) and fake_gguf.dequantize_tensor is patched
    gd.uninstall()
    assert fake_gguf.dequantize_tensor is orig_dq and fake_gguf.GGMLLayer.get_weight is orig_gw


def test_flag_off_means_no_patch(gd, fake_gguf, monkeypatch):
    monkeypatch.setenv("WEIGHTFERRY_GGUF_TRITON", "0")
    orig = fake_gguf.dequantize_tensor
    assert gd.install() is False and fake_gguf.dequantize_tensor is orig
    assert gd.install(force=True) is True                       # force overrides the flag


def test_without_gguf_module_nothing_happens(gd):
    assert gd.install(force=True) is False


def test_cpu_tensor_falls_back_to_host_code(gd, fake_gguf):
    gd.install(force=True)
    t = fake_gguf.GGMLTensor(torch.zeros(144, dtype=torch.uint8), tensor_type=12, tensor_shape=torch.Size((256,)))
    assert fake_gguf.dequantize_tensor(t, torch.bfloat16, None) == "host-dequant"
    assert gd.stats() == {"used": 0, "fallback": 1}
    assert fake_gguf.calls[-1][0] == "dequantize_tensor"


def test_unsupported_type_and_bad_dequant_dtype_fall_back(gd, fake_gguf):
    gd.install(force=True)
    t = fake_gguf.GGMLTensor(torch.zeros(16, dtype=torch.uint8), tensor_type=1, tensor_shape=torch.Size((8,)))
    assert fake_gguf.dequantize_tensor(t, torch.bfloat16, None) == "host-dequant"           # F16 type: not ours
    t = fake_gguf.GGMLTensor(torch.zeros(144, dtype=torch.uint8), tensor_type=12, tensor_shape=torch.Size((256,)))
    assert fake_gguf.dequantize_tensor(t, torch.bfloat16, "garbage") == "host-dequant"
    assert gd.stats()["fallback"] == 2 and gd.stats()["used"] == 0


def test_exception_is_logged_and_counted_twice(gd, fake_gguf, monkeypatch, caplog):
    gd.install(force=True)

    def boom(*a, **k):
        raise RuntimeError("kernel exploded")
    monkeypatch.setattr(gd, "dequantize", boom)
    t = fake_gguf.GGMLTensor(torch.zeros(144, dtype=torch.uint8), tensor_type=12, tensor_shape=torch.Size((256,)))
    with caplog.at_level("WARNING", logger="WeightFerry"):
        assert fake_gguf.dequantize_tensor(t, torch.bfloat16, None) == "host-dequant"
    assert "kernel exploded" in caplog.text
    assert gd.stats()["fallback"] == 2        # the reference counts the exception and the fallback (:532,538)


def test_kquant_gate(gd):
    gd._KQUANTS = False
    assert gd._supported(8) and not gd._supported(12)
    gd._KQUANTS = True
    assert gd._supported(12) and gd._supported(14) and not gd._supported(1)


def test_stats_reset(gd):
    gd._counts["used"] = 5
    assert gd.stats(reset=True)["used"] == 5
    assert gd.stats() == {"used": 0, "fallback": 0}


class LoRAAdapter:
    def __init__(self, weights):
        self.weights = weights


def _patch(up, down, alpha=None, strength=1.0, **over):
    w = [up, down, alpha, None, None, None]
    for k, v in over.items():
        w[int(k[1:])] = v
    return (strength, LoRAAdapter(tuple(w)), 1.0, None, None)


def test_lora_factors_eligibility(gd):
    up, down = torch.zeros(8, 4), torch.zeros(4, 16)
    got = gd.lora_factors([_patch(up, down, alpha=2.0, strength=0.5)], 8, 16)
    assert len(got) == 1 and got[0][0] is up and got[0][1] is down and got[0][2] == 0.5 * (2.0 / 4)
    assert gd.lora_factors([_patch(up, down)], 8, 16)[0][2] == 1.0          # alpha None -> 1
    assert gd.lora_factors([_patch(up, down, w3=torch.zeros(1))], 8, 16) is None      # DoRA scale
    assert gd.lora_factors([_patch(up, down)], 9, 16) is None                          # shape
    assert gd.lora_factors([_patch(up, down, strength=True)], 8, 16) is None           # bool strength
    assert gd.lora_factors([_patch(up, down, alpha="x")], 8, 16) is None
    assert gd.lora_factors([(1.0, LoRAAdapter((up, down, None, None, None, None)), 0.5, None, None)], 8, 16) is None
    assert gd.lora_factors([(1.0, object(), 1.0, None, None)], 8, 16) is None
    assert gd.lora_factors(["not a tuple"], 8, 16) is None
    assert gd.lora_factors([], 8, 16) == []


def test_get_weight_counts_lora_fallback(gd, fake_gguf):
    gd.install(force=True)
    layer = fake_gguf.GGMLLayer()
    up, down = torch.zeros(8, 4), torch.zeros(4, 16)
    t = fake_gguf.GGMLTensor(torch.zeros(10, dtype=torch.uint8), tensor_type=12, tensor_shape=torch.Size((8, 16)),
                             patches=[([_patch(up, down)], "key")])
    t.is_cuda_override = True
    # CPU tensor: not eligible, no LoRA counting, ComfyUI-GGUF's get_weight runs
    assert layer.get_weight(t, torch.bfloat16) == "host-get-weight"
    assert "lora_fallback" not in gd.stats()
    assert layer.get_weight(None, torch.bfloat16) is None


def test_version_of_inference_tensor_is_none(gd):
    # ComfyUI builds its tensors under torch.inference_mode: they have no version counter, and reading it raises
    with torch.inference_mode():
        t = torch.zeros(4, 4)
    with pytest.raises(RuntimeError):
        t._version
    assert gd._version(t) is None
    assert gd._version(torch.zeros(2)) == 0


def test_pinned_factor_of_inference_tensor_is_reused_then_released(gd, monkeypatch):
    # the page-locked copy is keyed by (storage, version, device); an inference-mode factor has version None and
    # must still be cached and reused, then forgotten when the factor is collected and released on request
    pinned_calls, emptied = [], []
    monkeypatch.setattr(torch.Tensor, "pin_memory", lambda self: pinned_calls.append(1) or self.clone())
    monkeypatch.setattr(torch._C, "_host_emptyCache", lambda: emptied.append(1), raising=False)
    store = gd._PinnedFactors()
    store._hooked = True                       # no ComfyUI here: nothing to hook
    with torch.inference_mode():
        up = torch.full((8, 4), 0.5, dtype=torch.bfloat16)
    a = store.upload(up, "cpu")
    b = store.upload(up, "cpu")
    assert a.dtype == torch.float32 and torch.equal(a, b) and len(pinned_calls) == 1 and len(store) == 1
    store.release()
    assert emptied == []                      # nothing dropped yet
    del up
    import gc
    gc.collect()
    assert len(store) == 0
    store.release()
    store.release()
    assert emptied == [1]


def test_comfy_memory_calls_release_pinned_copies(gd, monkeypatch):
    import types
    import sys
    calls = []
    mm = types.ModuleType("comfy.model_management")
    mm.free_memory = lambda *a, **k: calls.append(("free_memory", a, k)) or "freed"
    mm.unload_all_models = lambda: calls.append(("unload_all_models",))
    mm.soft_empty_cache = lambda force=False: calls.append(("soft_empty_cache", force))
    comfy = types.ModuleType("comfy")
    comfy.model_management = mm
    monkeypatch.setitem(sys.modules, "comfy", comfy)
    monkeypatch.setitem(sys.modules, "comfy.model_management", mm)
    emptied = []
    monkeypatch.setattr(torch._C, "_host_emptyCache", lambda: emptied.append(1), raising=False)
    monkeypatch.setattr(gd._PINNED, "_hooked", False)
    gd._hook_comfy_memory()
    gd._hook_comfy_memory()                    # once only: no double wrapping
    assert all(getattr(mm, n)._weightferry_cache for n in ("free_memory", "unload_all_models", "soft_empty_cache"))
    assert not getattr(mm.free_memory.__wrapped__, "_weightferry_cache", False)
    monkeypatch.setattr(gd._PINNED, "_freed", True)
    assert mm.free_memory(3, "cuda", keep=1) == "freed"
    assert emptied == [1] and calls[-1] == ("free_memory", (3, "cuda"), {"keep": 1})
    mm.soft_empty_cache(True)
    mm.unload_all_models()
    assert emptied == [1] and [c[0] for c in calls] == ["free_memory", "soft_empty_cache", "unload_all_models"]

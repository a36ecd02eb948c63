"""The WeightFerryDiT node's host side without a GPU: the reference's option names, choice strings and defaults
(streaming/dit_node.py:35-169 of the reference), the registration under the reference's node name, and the paths
that register nothing (disabled, a device that is not CUDA, every block resident)."""
import pytest

from conftest import sub

import fake_comfy


@pytest.fixture
def comfy():
    fake_comfy.make_comfy_modules()
    yield
    fake_comfy.remove_comfy_modules()


def test_option_names_and_defaults(pkg):
    node = sub("streaming.node")
    it = node.WeightFerryDiT.INPUT_TYPES()
    assert list(it["required"]) == ["model", "enabled", "pin_memory", "buffer_mode", "resident_blocks",
                                    "sage_attention"]
    assert list(it["optional"]) == ["host_format", "tiering", "ram_budget_gb", "resident_mode", "sage_pv_fp16",
                                    "auto_config", "prefetch_slots", "vram_budget_gb"]
    assert it["required"]["buffer_mode"][0] == ["Double Buffer (Async Prefetch, Recommended)",
                                                "Single Buffer (Synchronous)"]
    assert it["optional"]["tiering"][0] == ["RAM (all streamed blocks pinned in RAM)", "Auto (GPU / RAM / SSD)"]
    assert it["required"]["resident_blocks"][1]["default"] == 8 and it["optional"]["prefetch_slots"][1]["default"] == 3
    assert node.WeightFerryDiT.RETURN_TYPES == ("MODEL",) and node.WeightFerryDiT.FUNCTION == "apply_streaming"
    assert pkg.NODE_CLASS_MAPPINGS["WeightFerryDiT"] is node.WeightFerryDiT


def _stack(n=4):
    syn = sub("streaming.synthetic")
    m = syn.WanLikeStack(n_blocks=n, dim=512, heads=4, ffn=1024, qtype=12)
    return m


def test_paths_that_register_nothing(comfy):
    node = sub("streaming.node").WeightFerryDiT()
    mp = fake_comfy.FakeModelPatcher(_stack(), load_device="cuda")
    assert node.apply_streaming(mp, enabled=False)[0] is mp
    out = node.apply_streaming(mp, resident_blocks=4)[0]       # every block resident
    assert out is not mp and not out.callbacks
    cpu = fake_comfy.FakeModelPatcher(_stack(), load_device="cpu")
    out = node.apply_streaming(cpu)[0]
    assert not out.callbacks and "wrappers" not in out.model_options["transformer_options"]


def test_registration(comfy):
    node = sub("streaming.node").WeightFerryDiT()
    mp = fake_comfy.FakeModelPatcher(_stack(), load_device="cuda")
    out = node.apply_streaming(mp, resident_blocks=1, auto_config=True, sage_attention=True)[0]
    assert out is not mp and not mp.callbacks               # the input patcher is untouched (cloned)
    assert len(out.callbacks["on_load"]) == 1 and len(out.callbacks["on_detach"]) == 1
    assert list(out.model_options["transformer_options"]["wrappers"]["diffusion_model"]) == ["weightferry_dit"]
    again = node.apply_streaming(out, resident_blocks=1)[0]  # applying twice keeps one wrapper under the key
    assert len(again.model_options["transformer_options"]["wrappers"]["diffusion_model"]["weightferry_dit"]) == 1

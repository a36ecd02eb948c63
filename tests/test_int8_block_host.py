"""CPU behaviour of the int8 block adapter (enhancers.int8_block) on the stand-in Cosmos block: which layers count as
plain int8 linears (_int8_proj_ok, enhancers/fused_int8.py:108-115 of the reference), the WEIGHTFERRY_FUSED_BLOCK
parts, install / uninstall of the three methods, and -- on CPU tensors, where no int8 kernel applies -- the patched
block computing exactly what the unpatched one computes (every part steps aside)."""
import pytest
import torch

import fake_cosmos
from conftest import sub

ib = sub("enhancers.int8_block")
fi = sub("enhancers.fused_int8")
fs = sub("enhancers.fused_state")


@pytest.fixture
def quant_ops():
    fake_cosmos.install_quant_ops()
    yield
    fake_cosmos.remove_quant_ops()


@pytest.fixture
def mod():
    m = fake_cosmos.module()
    yield m
    ib.uninstall()


def test_proj_ok_rules(quant_ops):
    g = torch.Generator().manual_seed(1)
    lin = fake_cosmos._int8(g, 16, 256, "cpu")
    assert fi._int8_proj_ok(lin)
    lin.pre_quant_scale = torch.ones(256)                   # AWQ smoothing: the input is changed first
    assert not fi._int8_proj_ok(lin)
    lin = fake_cosmos._int8(g, 16, 256, "cpu")
    lin.quant_format = "fp8_scaled"                         # a format that quantises its input itself
    assert not fi._int8_proj_ok(lin)
    lin = fake_cosmos._int8(g, 16, 256, "cpu")
    lin.forward = lambda x: x                               # a forward of its own on the instance
    assert not fi._int8_proj_ok(lin)
    assert not fi._int8_proj_ok(torch.nn.Linear(4, 4))      # no _forward, not int8


def test_proj_ok_without_comfy_is_false():
    g = torch.Generator().manual_seed(1)
    assert not fi._int8_proj_ok(fake_cosmos._int8(g, 16, 256, "cpu"))


def test_wanted_parts(monkeypatch):
    monkeypatch.setenv("WEIGHTFERRY_FUSED_BLOCK", "0")
    assert ib.wanted_parts() == ()
    monkeypatch.setenv("WEIGHTFERRY_FUSED_BLOCK", "1")
    assert ib.wanted_parts() == ib.PARTS
    monkeypatch.setenv("WEIGHTFERRY_FUSED_BLOCK", "res, gelu,nonsense")
    assert ib.wanted_parts() == ("gelu", "res")


def test_install_and_uninstall(mod):
    orig = (mod.Block.forward, mod.Attention.compute_qkv, mod.GPT2FeedForward.forward)
    assert ib.install(module=mod) == ib.PARTS
    assert mod.Block.forward is ib._block_forward and mod.Attention.compute_qkv is ib._compute_qkv
    assert mod.GPT2FeedForward.forward is ib._mlp_forward
    assert ib.install(("res",), module=mod) == ("res",)     # qkv off: ComfyUI's compute_qkv back
    assert mod.Attention.compute_qkv is orig[1] and mod.GPT2FeedForward.forward is orig[2]
    assert ib.install(("ln", "qkv"), module=mod) == ("qkv",)   # ln needs modq
    ib.uninstall()
    assert (mod.Block.forward, mod.Attention.compute_qkv, mod.GPT2FeedForward.forward) == orig


def test_cpu_block_equals_unpatched(quant_ops, mod):
    torch.manual_seed(0)
    blk = fake_cosmos.Block(dim=256, heads=2, hidden=512, context_dim=256, seed=3, device="cpu")
    g = torch.Generator().manual_seed(5)
    x = torch.randn((1, 2, 4, 4, 256), generator=g).to(torch.bfloat16)
    emb = torch.randn((1, 2, 256), generator=g).to(torch.bfloat16)
    ctx = torch.randn((1, 7, 256), generator=g).to(torch.bfloat16)
    with torch.no_grad():
        ref = blk(x, emb, ctx)
        ib.install(module=mod)
        fs.stats(reset=True)
        got = blk(x, emb, ctx)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    st = fs.stats()
    # nothing ran on the kernels: CPU inputs are not the int8 path's case
    assert all(v["used"] == 0 for v in st.values()) and st["qkv"]["fallback"] > 0

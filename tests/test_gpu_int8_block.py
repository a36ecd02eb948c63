"""The int8 path driven by its block adapter (enhancers.int8_block) on the GPU, on the stand-in Cosmos-Predict2 block
(tests/fake_cosmos.py) whose int8 linears, when not overridden, run ComfyUI's own order: quantise the real input
(ConvRot), int8 GEMM to bf16.

* With every part on, the block's output equals, bit for bit, the oracle's composition of the same fused steps:
  LayerNorm + scale-and-shift inside the q / k / v, cross-attention q and MLP layer1 quantisers (one quantisation
  shared by q / k / v), GELU inside MLP layer2's quantiser, the three residual adds in the output projections'
  epilogues, every int8 step by the oracle and only the attention itself (torch SDPA on the same q / k / v) and the
  AdaLN modulations by torch.
* Without the LayerNorm part, the block's output equals the unpatched block's bit for bit: the pending
  scale-and-shift, the shared quantisation, the GELU table and the residual epilogue give ComfyUI's own bits.
* The used / fallback counters show every part running.
"""
import numpy as np
import pytest
import torch

import fake_cosmos
from conftest import sub
from oracle import lib

pytestmark = pytest.mark.gpu

ib = sub("enhancers.int8_block")
fi = sub("enhancers.fused_int8")
fs = sub("enhancers.fused_state")

B, T, H, W, D, HID, CTX, CD = 2, 2, 4, 16, 512, 1024, 77, 256


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def _from_bits(bits, shape):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).reshape(shape).cuda()


def _plain_int8(layer, x, weight, bias):
    """ComfyUI's int8 ConvRot linear on the real input (quantise, then the GEMM), on the kernels."""
    out = fi.int8_linear(x, weight._qdata, weight._params.scale, convrot=True)
    assert out is not None
    return out


@pytest.fixture
def setup():
    fake_cosmos.install_quant_ops()
    fake_cosmos.LINEAR["fn"] = _plain_int8
    mod = fake_cosmos.module()
    blk = fake_cosmos.Block(dim=D, heads=4, hidden=HID, context_dim=CD, seed=11, device="cuda")
    g = torch.Generator().manual_seed(99)
    x = torch.randn((B, T, H, W, D), generator=g).to(torch.bfloat16).cuda()
    emb = torch.randn((B, T, D), generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn((B, CTX, CD), generator=g).to(torch.bfloat16).cuda()
    yield mod, blk, x, emb, ctx
    ib.uninstall()
    fake_cosmos.LINEAR["fn"] = fake_cosmos._default_linear
    fake_cosmos.remove_quant_ops()


def _o_linear(xq, xs, layer):
    w = layer.weight
    return lib.linear_i8(xq, w._qdata.cpu().numpy(), xs, w._params.scale.cpu().numpy(), out_dt=lib.BF16)


def _o_residual(xq, xs, layer, gate, resid):
    """oracle: resid + gate * linear, gate (B, T, 1, 1, D) per group of H * W rows"""
    w = layer.weight
    return lib.linear_i8_residual(xq, w._qdata.cpu().numpy(), xs, w._params.scale.cpu().numpy(),
                                  _bits(gate.reshape(B * T, D)), _bits(resid.reshape(-1, D)), H * W)


def _o_lnmod(x, scale, shift, eps=1e-6):
    s1 = (1 + scale).contiguous().reshape(B * T, D)
    return lib.quant_rows_pre(_bits(x.reshape(-1, D)), 3, _bits(s1), _bits(shift.reshape(B * T, D)), H * W, eps)


def _attend(attn, q, k, v):
    """the stand-in's own attention on bf16 q / k / v [b, s, D] (split into heads as its compute_qkv does), before
    the output projection"""
    return attn.attend(*(t.reshape(t.shape[0], t.shape[1], attn.n_heads, attn.head_dim) for t in (q, k, v)))


def _oracle_block(blk, x, emb, ctx):
    mods = []
    for layer in (blk.adaln_modulation_self_attn, blk.adaln_modulation_cross_attn, blk.adaln_modulation_mlp):
        mods.append([t.unsqueeze(2).unsqueeze(2) for t in layer(emb).chunk(3, dim=-1)])
    (sh_sa, sc_sa, g_sa), (sh_ca, sc_ca, g_ca), (sh_mlp, sc_mlp, g_mlp) = mods
    tok = (B, T * H * W, D)
    sa, ca, mlp = blk.self_attn, blk.cross_attn, blk.mlp
    # self-attention: one LayerNorm + scale-and-shift quantisation shared by q, k, v
    xq, xs = _o_lnmod(x, sc_sa, sh_sa)
    q, k, v = (_from_bits(_o_linear(xq, xs, p), tok) for p in (sa.q_proj, sa.k_proj, sa.v_proj))
    a = _attend(sa, q, k, v)
    aq, as_ = lib.quant_rows(_bits(a.reshape(-1, D)), 1)
    x = _from_bits(_o_residual(aq, as_, sa.output_proj, g_sa, x), x.shape)
    # cross-attention: q from the pending input, k / v from the context the plain way
    xq, xs = _o_lnmod(x, sc_ca, sh_ca)
    q = _from_bits(_o_linear(xq, xs, ca.q_proj), tok)
    cq, cs = lib.quant_rows(_bits(ctx.reshape(-1, CD)), 1)
    k, v = (_from_bits(_o_linear(cq, cs, p), (B, CTX, D)) for p in (ca.k_proj, ca.v_proj))
    a = _attend(ca, q, k, v)
    aq, as_ = lib.quant_rows(_bits(a.reshape(-1, D)), 1)
    x = _from_bits(_o_residual(aq, as_, ca.output_proj, g_ca, x), x.shape)
    # MLP: layer1 from the pending input, GELU inside layer2's quantiser, residual in layer2's epilogue
    xq, xs = _o_lnmod(x, sc_mlp, sh_mlp)
    h = _o_linear(xq, xs, mlp.layer1)
    table = torch.nn.functional.gelu(torch.arange(65536, dtype=torch.int32, device="cuda").to(torch.int16)
                                     .view(torch.bfloat16))
    hq, hs = lib.quant_rows_pre(h, 1, _bits(table))
    return _from_bits(_o_residual(hq, hs, mlp.layer2, g_mlp, x), x.shape)


def test_all_parts_equal_the_oracles_composition(setup):
    mod, blk, x, emb, ctx = setup
    assert ib.install(module=mod) == ib.PARTS
    fs.stats(reset=True)
    with torch.no_grad():
        got = blk(x, emb, ctx)
        torch.cuda.synchronize()
        st = fs.stats()
        ref = _oracle_block(blk, x, emb, ctx)
    torch.cuda.synchronize()
    bad = np.argwhere(_bits(got) != _bits(ref))
    assert bad.size == 0, (len(bad), bad[:6].tolist())
    # every part ran: three LayerNorm + scale-and-shift inputs, one GELU, three residual epilogues; q / k / v,
    # cross q, both output projections and both MLP layers through the shared path
    assert st["ln"] == {"used": 3, "fallback": 0, "why": None}, st
    assert st["gelu"]["used"] == 1 and st["res"]["used"] == 3 and st["qkv"]["fallback"] == 0, st
    assert "modq" not in st or st["modq"]["fallback"] == 0


@pytest.mark.parametrize("parts", [("qkv", "modq", "gelu", "res"), ("qkv", "res"), ("gelu",), ("qkv", "modq")])
def test_without_layernorm_equals_the_unpatched_block(setup, parts):
    mod, blk, x, emb, ctx = setup
    with torch.no_grad():
        ref = blk(x, emb, ctx)
        torch.cuda.synchronize()
        assert ib.install(parts, module=mod) == parts
        fs.stats(reset=True)
        got = blk(x, emb, ctx)
    torch.cuda.synchronize()
    bad = np.argwhere(_bits(got) != _bits(ref))
    assert bad.size == 0, (parts, len(bad), bad[:6].tolist())
    st = fs.stats()
    if "res" in parts:
        assert st["res"]["used"] == 3, st
    if "modq" in parts:
        assert st["modq"]["used"] == 3 and st["modq"]["fallback"] == 0, st
    if "gelu" in parts:
        assert st["gelu"]["used"] == 1, st


def test_merged_gates_for_equal_rows(setup):
    # classifier-free guidance: every (batch, frame) row of the modulation input equal -> one residual GEMM over all
    # rows with one gate row (WEIGHTFERRY_CFG_RESID_MERGE), the same bits as one gate row per group
    mod, blk, x, emb, ctx = setup
    emb = emb[:1, :1].expand(B, T, D).contiguous()
    fi._VERIFY_GATES = True
    try:
        with torch.no_grad():
            ref = blk(x, emb, ctx)
            ib.install(module=mod)
            ib._MERGE_GATES = True
            fs.stats(reset=True)
            got = blk(x, emb, ctx)
            ib._MERGE_GATES = False
            emb2 = emb.clone()          # a fresh tensor: the row check runs again
            split = blk(x, emb2, ctx)
        torch.cuda.synchronize()
    finally:
        fi._VERIFY_GATES = False
        ib._MERGE_GATES = None
    st = fs.stats()
    assert st["resmerge"]["used"] == 3 and st["resmerge_gate"]["fallback"] == 0, st
    assert torch.equal(got.view(torch.int16), split.view(torch.int16))
    # with the LayerNorm in the quantisers the fused block is not compared with the unpatched one here
    assert got.shape == ref.shape

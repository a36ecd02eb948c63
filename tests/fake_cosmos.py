"""Stand-ins for the parts of ComfyUI that the int8 block adapter patches and reads, built the way ComfyUI builds
them (comfy/ldm/cosmos/predict2.py, comfy/quant_ops.py), small enough for tests:

* ``install_quant_ops()`` registers ``comfy.quant_ops`` with QUANT_ALGOS (one int8 format whose input the layer
  does not quantise itself), QuantizedTensor (the FakeQT of fake_quant) and TensorWiseINT8Layout.get_plain_tensors;
* ``Int8Linear`` -- ComfyUI's quantised linear: ``forward`` calls ``self._forward(input, weight, bias)``; its class
  ``_forward`` is ComfyUI's own int8 path (``LINEAR`` below: quantise the real input, int8 GEMM);
* ``Attention``, ``GPT2FeedForward``, ``Block`` -- the Cosmos-Predict2 block: AdaLN modulations, three LayerNorms
  without affine parameters, self-attention (q, k, v, output projections), cross-attention on a context, MLP
  (layer1, GELU, layer2), every sub-layer added to the residual stream with ``torch.addcmul``.
"""
import sys
import types

import torch

from fake_quant import FakeQT

INT8_FORMAT = "int8_tensorwise"


def install_quant_ops():
    comfy = sys.modules.get("comfy") or types.ModuleType("comfy")
    qo = types.ModuleType("comfy.quant_ops")
    qo.QUANT_ALGOS = {INT8_FORMAT: {"quantize_input": False}, "fp8_scaled": {"quantize_input": True}}
    qo.QuantizedTensor = FakeQT

    class TensorWiseINT8Layout:
        @staticmethod
        def get_plain_tensors(qt):
            return qt._qdata, qt._params.scale
    qo.TensorWiseINT8Layout = TensorWiseINT8Layout
    comfy.quant_ops = qo
    sys.modules["comfy"] = comfy
    sys.modules["comfy.quant_ops"] = qo
    return qo


def remove_quant_ops():
    sys.modules.pop("comfy.quant_ops", None)
    comfy = sys.modules.get("comfy")
    if comfy is not None and hasattr(comfy, "quant_ops"):
        del comfy.quant_ops
        if not any(k.startswith("comfy.") for k in sys.modules):
            sys.modules.pop("comfy", None)


def _default_linear(layer, x, weight, bias):
    return torch.nn.functional.linear(x, weight, bias)


# ComfyUI's own int8 linear (no _forward override): a test sets it to the computation it stands for
LINEAR = {"fn": _default_linear}


class Int8Linear(torch.nn.Module):
    def __init__(self, w_q, scale, quant_format=INT8_FORMAT):
        super().__init__()
        self.weight = FakeQT(w_q, scale)
        self.bias = None
        self.quant_format = quant_format
        self.in_features, self.out_features = w_q.shape[1], w_q.shape[0]

    def _forward(self, input, weight, bias):
        return LINEAR["fn"](self, input, weight, bias)

    def forward(self, x):
        return self._forward(x, self.weight, self.bias)


def _int8(g, n, k, device):
    w_q = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int64).to(torch.int8)
    ws = torch.rand(n, generator=g) * 0.004 + 0.001
    return Int8Linear(w_q.to(device), ws.to(device))


class Attention(torch.nn.Module):
    def __init__(self, g, dim, heads, context_dim, selfattn, device):
        super().__init__()
        self.is_selfattn, self.n_heads, self.head_dim = selfattn, heads, dim // heads
        self.q_proj = _int8(g, dim, dim, device)
        self.k_proj = _int8(g, dim, context_dim, device)
        self.v_proj = _int8(g, dim, context_dim, device)
        self.output_proj = _int8(g, dim, dim, device)
        self.output_dropout = torch.nn.Identity()

    def compute_qkv(self, x, context=None, rope_emb=None, transformer_options={}):
        q = self.q_proj(x)
        ctx = x if context is None else context
        k, v = self.k_proj(ctx), self.v_proj(ctx)
        return tuple(t.reshape(*t.shape[:-1], self.n_heads, self.head_dim) for t in (q, k, v))

    def attend(self, q, k, v):
        """softmax attention of q [b, s, h, d] over k / v [b, s', h, d] -> [b, s, h d]"""
        b, s = q.shape[:2]
        q, k, v = (t.transpose(1, 2).contiguous() for t in (q, k, v))
        out = torch.nn.functional.scaled_dot_product_attention(q, k, v)
        return out.transpose(1, 2).reshape(b, s, -1)

    def compute_attention(self, q, k, v, transformer_options={}):
        return self.output_dropout(self.output_proj(self.attend(q, k, v)))

    def forward(self, x, context=None, rope_emb=None, transformer_options={}):
        q, k, v = self.compute_qkv(x, context, rope_emb=rope_emb, transformer_options=transformer_options)
        return self.compute_attention(q, k, v, transformer_options=transformer_options)


class GPT2FeedForward(torch.nn.Module):
    def __init__(self, g, dim, hidden, device):
        super().__init__()
        self.layer1 = _int8(g, hidden, dim, device)
        self.activation = torch.nn.GELU()
        self.layer2 = _int8(g, dim, hidden, device)

    def forward(self, x):
        return self.layer2(self.activation(self.layer1(x)))


class Block(torch.nn.Module):
    def __init__(self, dim=512, heads=4, hidden=1024, context_dim=256, seed=0, device="cuda"):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.self_attn = Attention(g, dim, heads, dim, True, device)
        self.cross_attn = Attention(g, dim, heads, context_dim, False, device)
        self.mlp = GPT2FeedForward(g, dim, hidden, device)
        self.layer_norm_self_attn = torch.nn.LayerNorm(dim, elementwise_affine=False, eps=1e-6)
        self.layer_norm_cross_attn = torch.nn.LayerNorm(dim, elementwise_affine=False, eps=1e-6)
        self.layer_norm_mlp = torch.nn.LayerNorm(dim, elementwise_affine=False, eps=1e-6)
        self.use_adaln_lora = False

        def adaln():
            lin = torch.nn.Linear(dim, 3 * dim, bias=False)
            lin.weight.data = (torch.randn((3 * dim, dim), generator=g) * 0.05).to(torch.bfloat16)
            return torch.nn.Sequential(torch.nn.SiLU(), lin).to(device)
        self.adaln_modulation_self_attn = adaln()
        self.adaln_modulation_cross_attn = adaln()
        self.adaln_modulation_mlp = adaln()

    def forward(self, x_B_T_H_W_D, emb_B_T_D, crossattn_emb, rope_emb_L_1_1_D=None, adaln_lora_B_T_3D=None,
                extra_per_block_pos_emb=None, transformer_options={}):
        x = x_B_T_H_W_D
        residual_dtype, compute_dtype = x.dtype, emb_B_T_D.dtype
        if extra_per_block_pos_emb is not None:
            x = x + extra_per_block_pos_emb
        mods = []
        for layer in (self.adaln_modulation_self_attn, self.adaln_modulation_cross_attn, self.adaln_modulation_mlp):
            m = layer(emb_B_T_D)
            if self.use_adaln_lora:
                m = m + adaln_lora_B_T_3D
            mods.append([t.unsqueeze(2).unsqueeze(2) for t in m.chunk(3, dim=-1)])
        (sh_sa, sc_sa, g_sa), (sh_ca, sc_ca, g_ca), (sh_mlp, sc_mlp, g_mlp) = mods
        B, T, H, W, D = x.shape

        def modulate(norm, t, scale, shift):
            return norm(t) * (1 + scale) + shift

        n = modulate(self.layer_norm_self_attn, x, sc_sa, sh_sa)
        r = self.self_attn(n.to(compute_dtype).reshape(B, T * H * W, D), None, rope_emb=rope_emb_L_1_1_D,
                           transformer_options=transformer_options).reshape(B, T, H, W, D)
        x = torch.addcmul(x, g_sa.to(residual_dtype), r.to(residual_dtype))
        n = modulate(self.layer_norm_cross_attn, x, sc_ca, sh_ca)
        r = self.cross_attn(n.to(compute_dtype).reshape(B, T * H * W, D), crossattn_emb, rope_emb=rope_emb_L_1_1_D,
                            transformer_options=transformer_options).reshape(B, T, H, W, D)
        x = torch.addcmul(x, g_ca.to(residual_dtype), r.to(residual_dtype))
        n = modulate(self.layer_norm_mlp, x, sc_mlp, sh_mlp)
        r = self.mlp(n.to(compute_dtype))
        return torch.addcmul(x, g_mlp.to(residual_dtype), r.to(residual_dtype))


def module():
    """A module object with the three classes, as comfy.ldm.cosmos.predict2 has them."""
    mod = types.ModuleType("fake_predict2")
    mod.Block, mod.Attention, mod.GPT2FeedForward = Block, Attention, GPT2FeedForward
    return mod

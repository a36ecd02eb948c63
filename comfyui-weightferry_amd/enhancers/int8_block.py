"""The int8 path's caller inside ComfyUI's Cosmos-Predict2 / Anima DiT block (comfy/ldm/cosmos/predict2.py).

ComfyUI's ``Block.forward`` runs three sub-layers (self-attention, cross-attention, MLP). Each one reads
``LayerNorm(x) * (1 + scale) + shift`` and adds ``gate * out`` to the residual stream ``x``; every intermediate is a
tensor in HBM, and each int8 projection quantises its own input. Installed, this module replaces ``Block.forward``,
``Attention.compute_qkv`` and ``GPT2FeedForward.forward`` so that the block's int8 linears go through ``fused_int8``
with these parts (``WEIGHTFERRY_FUSED_BLOCK``: "1" all, "0" none, or a comma-separated list):

* ``qkv``  -- q, k and v of the self-attention share one quantisation of their common input;
* ``modq`` -- the scale-and-shift is not computed: the input projections' quantiser applies it;
* ``ln``   -- the LayerNorm before it is not computed either (needs ``modq``; widths that are powers of two and
  multiples of 512);
* ``gelu`` -- the MLP's GELU is applied by its second layer's quantiser;
* ``res``  -- ``x + gate * out`` is computed in the output projection's GEMM epilogue.

Every part is checked per call and steps aside when its case is not met, so the block then computes what ComfyUI
computes: an input no projection took is computed the plain way and the sub-layer is run again on it, a residual no
epilogue added is added with ComfyUI's ``torch.addcmul``. The reference's fused block
(enhancers/fused_block.py:424-735) has the same parts for this path; its Triton element-wise kernels,
SageAttention and TaylorSeer parts are outside it.
"""
import weakref
from collections import namedtuple

import torch

from ..core import env as _env
from ..utils.logging import log_info, log_warn
from .fused_int8 import _clear_pre, _int8_proj_ok, _Overrides, _residual_forward, _set_pre
from .fused_state import _count, _state, _tls

PARTS = ("qkv", "modq", "ln", "gelu", "res")
_MERGE_GATES = None   # None: WEIGHTFERRY_CFG_RESID_MERGE decides per forward; True / False force it
_PENDING_PART = {"lnmod": "ln", "mod": "modq", "gelu": "gelu"}


def wanted_parts():
    """The parts WEIGHTFERRY_FUSED_BLOCK names: every part for "1" / "on" / "true" / "all" or when unset, none for
    "0" / "off" / "false", else the listed ones (in PARTS order; unknown names are ignored)."""
    flag = (_env.get("WEIGHTFERRY_FUSED_BLOCK") or "1").strip().lower()
    if flag in ("", "0", "off", "false"):
        return ()
    if flag in ("1", "on", "true", "all"):
        return PARTS
    named = {p.strip() for p in flag.split(",")}
    return tuple(p for p in PARTS if p in named)


def _on(*parts):
    return all(p in _state["parts"] for p in parts)


# ------------------------------------------------------------------------------------------ eligibility
def _unpatched(module, *methods):
    """No instance-level override of ``methods`` on ``module`` (another node's patch would see our tensors)."""
    return not any(m in module.__dict__ for m in methods)


def _bf16_cuda(t):
    return t.dtype == torch.bfloat16 and t.is_cuda and t.is_contiguous()


def _plain_layernorm(norm, width):
    """ComfyUI's LayerNorm over the last dimension with no affine parameters and nothing for its cast path to apply,
    at a width the quantiser's LayerNorm splits into rows as PyTorch's kernel does (a power of two, a multiple of
    512)."""
    return (isinstance(norm, torch.nn.LayerNorm) and _unpatched(norm, "forward")
            and norm.weight is None and norm.bias is None and tuple(norm.normalized_shape) == (width,)
            and width % 512 == 0 and width & (width - 1) == 0
            and not getattr(norm, "weight_function", ()) and not getattr(norm, "bias_function", ()))


class _BlockCall:
    """What one call of the block may fuse, settled once per call. A pending input needs the qkv and modq parts, no
    transformer patches (they would see the normalised input), a bf16 block, ComfyUI's own attention and MLP
    methods, and every input projection -- self-attention q / k / v, cross-attention q, MLP layer1 -- a plain int8
    linear; the same facts decide the residual epilogue's part of it."""

    def __init__(self, block, transformer_options, compute_dtype, residual_dtype):
        self.patched = bool((transformer_options or {}).get("patches"))
        self.compute_dtype, self.residual_dtype = compute_dtype, residual_dtype
        sa, ca, mlp = block.self_attn, block.cross_attn, block.mlp
        self.pending = (_on("qkv", "modq") and not self.patched and compute_dtype == torch.bfloat16
                        and _unpatched(sa, "forward", "compute_qkv") and _unpatched(ca, "forward", "compute_qkv")
                        and _unpatched(mlp, "forward")
                        and all(_int8_proj_ok(p) for p in (sa.q_proj, sa.k_proj, sa.v_proj, ca.q_proj, mlp.layer1)))
        self.same_gate = False

    def input_forms(self, norm, x, scale, shift):
        """The sub-layer's input in the forms to try, best first, as (pending kind or None, tensor the module
        receives): x with LayerNorm and scale-and-shift pending, norm(x) with the scale-and-shift pending, and the
        real input. norm(x) is computed only when the first form is not taken."""
        if self.pending and _on("ln") and _bf16_cuda(x) and _plain_layernorm(norm, x.shape[-1]):
            yield "lnmod", x
        normed = norm(x)
        if self.pending and _bf16_cuda(normed):
            yield "mod", normed
        yield None, normed * (1 + scale) + shift

    def epilogue_ok(self, out_proj, x):
        return (_on("res") and not self.patched and out_proj is not None and _int8_proj_ok(out_proj)
                and x.dtype == self.compute_dtype)


# -------------------------------------------------------------------------------------------- sub-layers
# One sub-layer of the block as data: its LayerNorm and modulation, ``run`` (the module on an input, reshaped back
# to the residual's layout), the projection that may add the residual, and input projections outside
# compute_qkv's shared quantisation that should take the pending input.
_Sub = namedtuple("_Sub", "module norm shift scale gate run out_proj shared")


def _with_epilogue(call, sub, x, inp):
    """sub.run(inp) with the sub's int8 projections computing through fused_int8, and ``x + gate * out`` left
    pending for the output projection's epilogue when allowed. Returns (out, whether the residual was added)."""
    res = None
    layers = list(sub.shared)
    if call.epilogue_ok(sub.out_proj, x):
        res = {"x": x, "gate": sub.gate, "done": False, "same": call.same_gate}
        layers.append((sub.out_proj, _residual_forward))
    _tls.res = res
    try:
        with _Overrides(layers):
            out = sub.run(inp)
    finally:
        _tls.res = None
    return out, res is not None and res["done"]


def _step(call, sub, x):
    """The residual stream after one sub-layer: the first input form some projection takes (an untaken pending
    form is counted as a fallback of its part and the next form tried), then the residual added in the epilogue
    or by ComfyUI's addcmul."""
    for kind, inp in call.input_forms(sub.norm, x, sub.scale, sub.shift):
        if kind is None:
            out, added = _with_epilogue(call, sub, x, inp)
            break
        pend = _set_pre(inp, kind, sub.scale, sub.shift, norm=sub.norm if kind == "lnmod" else None)
        try:
            out, added = _with_epilogue(call, sub, x, inp)
        finally:
            _clear_pre()
        if pend.used:
            break
        _count(_PENDING_PART[kind], False, f"{type(sub.module).__name__} did not take the pending input")
    if added:
        return out
    rd = call.residual_dtype
    return torch.addcmul(x, sub.gate.to(rd), out.to(rd))


def _equal_gate_rows(emb, lora):
    """WEIGHTFERRY_CFG_RESID_MERGE: whether every (batch, frame) row of the modulation input -- timestep embedding
    and AdaLN-LoRA term -- is the same, so that every gate row is (classifier-free guidance batches share the
    timestep) and the residual epilogue can run once over all rows with one gate row. One device-to-host sync per
    forward: the answer is kept for the embedding object ComfyUI hands to every block, through weak references, so
    a later tensor at the same address is never taken for it."""
    memo = getattr(_tls, "gate_rows", None)
    if memo is not None and memo[0]() is emb and (memo[1]() if memo[1] is not None else None) is lora:
        return memo[2]

    def uniform(t):
        if t is None:
            return True
        return t.dim() == 3 and bool((t == t[:1, :1]).all())
    same = emb.dim() == 3 and emb.shape[0] * emb.shape[1] > 1 and uniform(emb) and uniform(lora)
    _tls.gate_rows = (weakref.ref(emb), weakref.ref(lora) if lora is not None else None, same)
    return same


# ------------------------------------------------------------------------------------- the patched methods
def _block_forward(self, x_B_T_H_W_D, emb_B_T_D, crossattn_emb, rope_emb_L_1_1_D=None, adaln_lora_B_T_3D=None,
                   extra_per_block_pos_emb=None, transformer_options={}):
    """ComfyUI's Block.forward (same signature), its three sub-layers run by ``_step``."""
    x, emb, lora = x_B_T_H_W_D, emb_B_T_D, adaln_lora_B_T_3D
    call = _BlockCall(self, transformer_options, emb.dtype, x.dtype)
    merge = _MERGE_GATES if _MERGE_GATES is not None else _env.get("WEIGHTFERRY_CFG_RESID_MERGE") == "1"
    call.same_gate = bool(merge and _on("res") and _equal_gate_rows(emb, lora))
    if extra_per_block_pos_emb is not None:
        x = x + extra_per_block_pos_emb
    # (shift, scale, gate) of each sub-layer, (B, T, 1, 1, D)
    mods = []
    for adaln in (self.adaln_modulation_self_attn, self.adaln_modulation_cross_attn, self.adaln_modulation_mlp):
        m = adaln(emb)
        if self.use_adaln_lora:
            m = m + lora
        mods.append([c[:, :, None, None, :] for c in m.chunk(3, dim=-1)])
    B, T, H, W, D = x.shape
    cd = call.compute_dtype

    def attention(attn, context):
        def run(n):
            out = attn(n.to(cd).reshape(B, T * H * W, D), context, rope_emb=rope_emb_L_1_1_D,
                       transformer_options=transformer_options)
            return out.reshape(B, T, H, W, D)
        return run

    sa, ca = self.self_attn, self.cross_attn
    x = _step(call, _Sub(sa, self.layer_norm_self_attn, *mods[0], attention(sa, None), sa.output_proj, ()), x)
    x = _step(call, _Sub(ca, self.layer_norm_cross_attn, *mods[1], attention(ca, crossattn_emb), ca.output_proj,
                         (ca.q_proj,)), x)
    shift, scale, gate = mods[2]
    patches = (transformer_options or {}).get("patches", {})
    if "mlp_patch" not in patches:
        return _step(call, _Sub(self.mlp, self.layer_norm_mlp, shift, scale, gate, lambda n: self.mlp(n.to(cd)),
                                self.mlp.layer2, ()), x)
    # ComfyUI's MLP patches see the real input: nothing pending, no epilogue
    args = {"x": (self.layer_norm_mlp(x) * (1 + scale) + shift).to(cd), "transformer_options": transformer_options}
    for patch in patches["mlp_patch"]:
        args = patch(args)
    out = self.mlp(args["x"])
    rd = call.residual_dtype
    return torch.addcmul(x, gate.to(rd), out.to(rd))


def _compute_qkv(self, x, context=None, rope_emb=None, transformer_options={}):
    """ComfyUI's Attention.compute_qkv; for the self-attention, its q / k / v projections compute through
    fused_int8 together, so their common input (or the pending one) is quantised once."""
    orig = _state["orig"]["compute_qkv"]
    shared = (context is None and getattr(self, "is_selfattn", False) and _on("qkv")
              and "attn1_patch" not in (transformer_options or {}).get("patches", {}))
    if shared:
        projs = [p for p in (self.q_proj, self.k_proj, self.v_proj) if hasattr(p, "_forward")]
        if len(projs) == 3:
            with _Overrides(projs):
                return orig(self, x, context, rope_emb=rope_emb, transformer_options=transformer_options)
        _count("qkv", False, "projections without _forward")
    return orig(self, x, context, rope_emb=rope_emb, transformer_options=transformer_options)


def _mlp_forward(self, x):
    """ComfyUI's GPT2FeedForward.forward (layer1, activation, layer2). layer1 takes the block's pending input, when
    there is one; with the gelu part, torch's exact GELU is left pending for layer2's quantiser. A pending input a
    layer did not take is computed the plain way and that layer run again on it."""
    orig = _state["orig"]["mlp_forward"]
    act = getattr(self, "activation", None)
    gelu = (_on("gelu") and type(act) is torch.nn.GELU and getattr(act, "approximate", "none") == "none"
            and _int8_proj_ok(self.layer2))
    inherited = getattr(_tls, "pre", None)          # the block's pending input for layer1
    if inherited is None and not gelu:
        return orig(self, x)
    with _Overrides([self.layer1, self.layer2]):
        h = self.layer1(x)
        if inherited is not None:
            _clear_pre()                            # the block's pending input ends at layer1
            if not inherited.used:
                _count("modq", False, "mlp.layer1 did not take the pending input")
                h = self.layer1(inherited.real().view(x.shape))
        if not (gelu and _bf16_cuda(h)):
            return self.layer2(self.activation(h))
        pend = _set_pre(h, "gelu")
        try:
            out = self.layer2(h)
        finally:
            _clear_pre()
        if pend.used:
            return out
        _count("gelu", False, "mlp.layer2 did not take the pending input")
        return self.layer2(self.activation(h))


# ------------------------------------------------------------------------------------------------ install
# (class, method, replacement, the parts any of which needs it)
_METHODS = (("Block", "forward", _block_forward, PARTS),
            ("Attention", "compute_qkv", _compute_qkv, ("qkv",)),
            ("GPT2FeedForward", "forward", _mlp_forward, ("gelu", "modq")))
_ORIG_KEY = {("Block", "forward"): "forward", ("Attention", "compute_qkv"): "compute_qkv",
             ("GPT2FeedForward", "forward"): "mlp_forward"}


def _cosmos_module():
    import comfy.ldm.cosmos.predict2 as p2
    return p2


def install(parts=None, module=None):
    """Replace the methods of ``module``'s Block / Attention / GPT2FeedForward (default: ComfyUI's
    comfy.ldm.cosmos.predict2) that ``parts`` (default: WEIGHTFERRY_FUSED_BLOCK) need, and give ComfyUI's back to
    the others; install(()) restores all three. Returns the parts in effect ("ln" only with "modq", which carries
    it)."""
    if module is None:
        try:
            module = _cosmos_module()
        except Exception as exc:  # noqa: BLE001 -- no ComfyUI Cosmos model: nothing to patch
            log_warn(f"int8 block: ComfyUI's Cosmos model not found ({exc}); not installed.")
            return ()
    chosen = set(wanted_parts() if parts is None else parts)
    if "modq" not in chosen:
        chosen.discard("ln")
    parts = tuple(p for p in PARTS if p in chosen)
    orig = _state.get("orig")
    if orig is None or orig.get("module") is not module:
        orig = {"module": module}
        for cls, meth, _fn, _needs in _METHODS:
            orig[_ORIG_KEY[(cls, meth)]] = getattr(getattr(module, cls), meth)
        _state["orig"] = orig
    _state["parts"] = parts
    for cls, meth, fn, needs in _METHODS:
        setattr(getattr(module, cls), meth, fn if set(parts) & set(needs) else orig[_ORIG_KEY[(cls, meth)]])
    if parts:
        log_info(f"int8 block: {', '.join(parts)} (WEIGHTFERRY_FUSED_BLOCK).")
    return parts


def uninstall():
    """ComfyUI's own methods back on the classes ``install`` patched."""
    orig = _state.get("orig")
    if orig is not None:
        install((), orig["module"])
    _state["parts"] = ()

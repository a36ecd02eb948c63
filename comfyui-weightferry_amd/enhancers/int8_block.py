"""The int8 path's caller inside ComfyUI's Cosmos-Predict2 / Anima DiT block (comfy/ldm/cosmos/predict2.py).

With int8 ConvRot weights, a block's three sub-layers (self-attention, cross-attention, MLP) each start from
``LayerNorm(x) * (1 + scale) + shift`` and end with ``x + gate * out``. ComfyUI writes every one of those
intermediate tensors and then quantises the projections' inputs one projection at a time. Installed, this module
replaces ``Block.forward``, ``Attention.compute_qkv`` and ``GPT2FeedForward.forward`` with versions that route the
block's int8 linears through ``fused_int8``:

* ``qkv``  -- the self-attention's q, k and v projections quantise their common input once;
* ``modq`` -- the scale-and-shift is left pending and the input projections' quantiser applies it;
* ``ln``   -- the LayerNorm before it as well (widths that are powers of two and multiples of 512);
* ``gelu`` -- the MLP's GELU is left pending for its second layer's quantiser;
* ``res``  -- ``x + gate * out`` is computed in the output projection's GEMM epilogue.

Every part checks its preconditions per call and otherwise leaves ComfyUI's computation in place: a pending
operation no layer took is computed the plain way, a residual no epilogue added is added with ``torch.addcmul``.
The parts and their order of operations are those of the reference's fused block (enhancers/fused_block.py:
320-345,424-524,589-700); its element-wise Triton kernels, SageAttention and TaylorSeer parts are not part of this
path. ``WEIGHTFERRY_FUSED_BLOCK`` selects the parts ("1": all, "0": none, or a comma-separated list).
"""
import torch

from ..core import env as _env
from ..utils.logging import log_info, log_warn
from .fused_int8 import (_clear_pre, _int8_proj_ok, _materialise, _Overrides, _residual_forward, _set_pre)
from .fused_state import _count, _state, _tls

PARTS = ("qkv", "modq", "ln", "gelu", "res")
_MERGE_GATES = None   # None: WEIGHTFERRY_CFG_RESID_MERGE decides per block; True / False force it


def wanted_parts():
    """The parts WEIGHTFERRY_FUSED_BLOCK asks for: all for "1" / "on" / "all" / unset, none for "0" / "off",
    else the listed ones."""
    flag = (_env.get("WEIGHTFERRY_FUSED_BLOCK") or "1").strip().lower()
    if flag in ("", "0", "off", "false"):
        return ()
    if flag in ("1", "on", "true", "all"):
        return PARTS
    asked = [p.strip() for p in flag.split(",")]
    return tuple(p for p in PARTS if p in asked)


def _on(part):
    return part in _state["parts"]


# -------------------------------------------------------------------------------------------- sub-layers
class _Call:
    """Facts of one block call that every sub-layer consults."""

    def __init__(self, block, transformer_options, compute_dtype, residual_dtype):
        self.block = block
        self.patched = bool((transformer_options or {}).get("patches"))
        self.compute_dtype = compute_dtype
        self.residual_dtype = residual_dtype

    def pending_allowed(self, tensor):
        """An input projection may take a pending scale-and-shift: modq and qkv on, no patches that would see
        the normalised input, bf16 all through, and every input projection of the block a plain int8 linear
        (enhancers/fused_block.py:489-502)."""
        if not (_on("modq") and _on("qkv")) or self.patched:
            return False
        if tensor.dtype != torch.bfloat16 or self.compute_dtype != torch.bfloat16:
            return False
        if not (tensor.is_cuda and tensor.is_contiguous()):
            return False
        blk = self.block
        sa, ca, mlp = blk.self_attn, blk.cross_attn, blk.mlp
        if any("forward" in m.__dict__ or "compute_qkv" in m.__dict__ for m in (sa, ca)) or "forward" in mlp.__dict__:
            return False
        return all(_int8_proj_ok(lin) for lin in (sa.q_proj, sa.k_proj, sa.v_proj, ca.q_proj, mlp.layer1))

    def norm_allowed(self, norm, x):
        """The LayerNorm may go into the quantiser: ComfyUI's LayerNorm without affine parameters and without
        cast functions, over the last dimension of a contiguous bf16 CUDA input whose width is a multiple of 512
        and a power of two (enhancers/fused_block.py:505-520)."""
        width = x.shape[-1]
        return (_on("ln") and isinstance(norm, torch.nn.LayerNorm) and "forward" not in norm.__dict__
                and norm.weight is None and norm.bias is None and len(norm.normalized_shape) == 1
                and width == norm.normalized_shape[0] and width % 512 == 0 and not width & (width - 1)
                and x.dtype == torch.bfloat16 and x.is_cuda and x.is_contiguous()
                and not getattr(norm, "weight_function", ()) and not getattr(norm, "bias_function", ()))


def _modulate(normed, scale, shift):
    """ComfyUI's scale-and-shift of a normalised input: normed * (1 + scale) + shift."""
    return normed * (1 + scale) + shift


def _run_sublayer(call, module, norm_and_x, scale, shift, fn, x_res, gate, out_layer, overrides=()):
    """fn(input) for one sub-layer whose input is ``norm(x) * (1 + scale) + shift`` (norm_and_x = (norm, x)):
    with that input left pending for the input projections' quantiser when allowed (LayerNorm included when
    allowed), and with ``x_res + gate * out`` inside out_layer's GEMM when allowed. Returns (out, residual added).
    A pending input no layer took is computed the plain way and the sub-layer runs again on it
    (enhancers/fused_block.py:523-567)."""
    with_res = (_on("res") and out_layer is not None and _int8_proj_ok(out_layer) and x_res is not None
                and x_res.dtype == call.compute_dtype and not call.patched)

    def run(inp):
        res = {"x": x_res, "gate": gate, "done": False, "same": getattr(_tls, "same_gate", False)} if with_res \
            else None
        _tls.res = res
        try:
            with _Overrides(list(overrides) + ([(out_layer, _residual_forward)] if with_res else [])):
                out = fn(inp)
        finally:
            _tls.res = None
        return out, bool(res is not None and res["done"])

    norm, x = norm_and_x
    if call.norm_allowed(norm, x) and call.pending_allowed(x):
        pre = _set_pre(x, "lnmod", scale, shift, norm=norm)
        try:
            got = run(x)
        finally:
            _clear_pre()
        if pre.used:
            return got
        _count("ln", False, f"{type(module).__name__} did not take the pending input")
    normed = norm(x)
    if call.pending_allowed(normed):
        pre = _set_pre(normed, "mod", scale, shift)
        try:
            got = run(normed)
        finally:
            _clear_pre()
        if pre.used:
            return got
        _count("modq", False, f"{type(module).__name__} did not take the pending input")
    return run(_modulate(normed, scale, shift))


def _join_residual(x_res, gate, out, added, residual_dtype):
    """The residual stream after a sub-layer: ``out`` itself when its GEMM already added x_res + gate * out,
    else ComfyUI's addcmul."""
    if added:
        return out
    return torch.addcmul(x_res, gate.to(residual_dtype), out.to(residual_dtype))


def _gates_equal(emb, lora):
    """Whether every (batch, frame) row of the block's modulation input is the same (classifier-free guidance
    batches share the timestep), so every gate row is: the residual epilogue then runs once over all rows with
    one gate row. One host sync per forward; cached on the embedding, which every block of a forward receives."""
    hit = getattr(emb, "_weightferry_rows_same", None)
    if hit is not None and hit[0] is lora:
        return hit[1]

    def rows_equal(t):
        return t is None or (t.dim() == 3 and bool(torch.equal(t, t[:1, :1].expand_as(t))))
    same = emb.dim() == 3 and emb.shape[0] * emb.shape[1] > 1 and rows_equal(emb) and rows_equal(lora)
    try:
        emb._weightferry_rows_same = (lora, same)
    except Exception:  # noqa: BLE001 -- an object that takes no attributes: checked again next block
        pass
    return same


# ------------------------------------------------------------------------------------------- the patched methods
def _block_forward(self, x_B_T_H_W_D, emb_B_T_D, crossattn_emb, rope_emb_L_1_1_D=None, adaln_lora_B_T_3D=None,
                   extra_per_block_pos_emb=None, transformer_options={}):
    """ComfyUI's Block.forward with its three sub-layers run through ``_run_sublayer``: the same operations in the
    same order wherever a part does not apply."""
    merge = _MERGE_GATES if _MERGE_GATES is not None else _env.get("WEIGHTFERRY_CFG_RESID_MERGE") == "1"
    _tls.same_gate = bool(merge and _on("res") and _gates_equal(emb_B_T_D, adaln_lora_B_T_3D))
    try:
        return _block_body(self, x_B_T_H_W_D, emb_B_T_D, crossattn_emb, rope_emb_L_1_1_D, adaln_lora_B_T_3D,
                           extra_per_block_pos_emb, transformer_options)
    finally:
        _tls.same_gate = False


def _modulation(block, emb, lora):
    """(shift, scale, gate) of each sub-layer as (B, T, 1, 1, D) tensors, from the block's AdaLN modulations."""
    out = []
    for layer in (block.adaln_modulation_self_attn, block.adaln_modulation_cross_attn, block.adaln_modulation_mlp):
        m = layer(emb)
        if block.use_adaln_lora:
            m = m + lora
        out.append(tuple(t.unsqueeze(2).unsqueeze(2) for t in m.chunk(3, dim=-1)))
    return out


def _block_body(self, x, emb, crossattn_emb, rope_emb, adaln_lora, extra_pos, transformer_options):
    call = _Call(self, transformer_options, emb.dtype, x.dtype)
    if extra_pos is not None:
        x = x + extra_pos
    (sh_sa, sc_sa, g_sa), (sh_ca, sc_ca, g_ca), (sh_mlp, sc_mlp, g_mlp) = _modulation(self, emb, adaln_lora)
    B, T, H, W, D = x.shape

    def tokens(n):                      # (B, T, H, W, D) -> (B, T H W, D), the attention's layout
        return n.to(call.compute_dtype).reshape(B, T * H * W, D)

    def grid(r):
        return r.reshape(B, T, H, W, D)

    out, added = _run_sublayer(
        call, self.self_attn, (self.layer_norm_self_attn, x), sc_sa, sh_sa,
        lambda n: self.self_attn(tokens(n), None, rope_emb=rope_emb, transformer_options=transformer_options),
        x, g_sa, self.self_attn.output_proj)
    x = _join_residual(x, g_sa, grid(out), added, call.residual_dtype)

    out, added = _run_sublayer(
        call, self.cross_attn, (self.layer_norm_cross_attn, x), sc_ca, sh_ca,
        lambda n: self.cross_attn(tokens(n), crossattn_emb, rope_emb=rope_emb,
                                  transformer_options=transformer_options),
        x, g_ca, self.cross_attn.output_proj, overrides=(self.cross_attn.q_proj,))
    x = _join_residual(x, g_ca, grid(out), added, call.residual_dtype)

    patches = (transformer_options or {}).get("patches", {})
    if "mlp_patch" in patches:
        normed = _modulate(self.layer_norm_mlp(x), sc_mlp, sh_mlp).to(call.compute_dtype)
        args = {"x": normed, "transformer_options": transformer_options}
        for patch in patches["mlp_patch"]:
            args = patch(args)
        out, added = self.mlp(args["x"]), False
    else:
        out, added = _run_sublayer(call, self.mlp, (self.layer_norm_mlp, x), sc_mlp, sh_mlp,
                                   lambda n: self.mlp(n.to(call.compute_dtype)), x, g_mlp, self.mlp.layer2)
    return _join_residual(x, g_mlp, out, added, call.residual_dtype)


def _compute_qkv(self, x, context=None, rope_emb=None, transformer_options={}):
    """ComfyUI's Attention.compute_qkv with the self-attention's three projections under one ``_Overrides``, so
    their common input is quantised once (and a pending input applied once)."""
    orig = _state["orig"]["compute_qkv"]
    if (context is not None or not getattr(self, "is_selfattn", False) or not _on("qkv")
            or "attn1_patch" in (transformer_options or {}).get("patches", {})):
        return orig(self, x, context, rope_emb=rope_emb, transformer_options=transformer_options)
    projs = [p for p in (self.q_proj, self.k_proj, self.v_proj) if hasattr(p, "_forward")]
    if len(projs) != 3:
        _count("qkv", False, "projections without _forward")
        return orig(self, x, context, rope_emb=rope_emb, transformer_options=transformer_options)
    with _Overrides(projs):
        return orig(self, x, context, rope_emb=rope_emb, transformer_options=transformer_options)


def _mlp_forward(self, x):
    """ComfyUI's GPT2FeedForward.forward (layer1, GELU, layer2) with a pending input taken by layer1 and the GELU
    left pending for layer2's quantiser."""
    orig = _state["orig"]["mlp_forward"]
    act = getattr(self, "activation", None)
    gelu_ok = (_on("gelu") and type(act) is torch.nn.GELU and getattr(act, "approximate", "none") == "none"
               and _int8_proj_ok(self.layer2))
    pre = getattr(_tls, "pre", None)
    if not gelu_ok and pre is None:
        return orig(self, x)
    with _Overrides([self.layer1, self.layer2]):
        h = self.layer1(x)
        if pre is not None:
            _clear_pre()
            if not pre.used:            # layer1 did not take the pending input: run it on the real one
                _count("modq", False, "mlp.layer1 did not take the pending input")
                h = self.layer1(_materialise(pre).view(x.shape))
        if not (gelu_ok and h.dtype == torch.bfloat16 and h.is_cuda and h.is_contiguous()):
            return self.layer2(self.activation(h))
        gelu = _set_pre(h, "gelu")
        try:
            out = self.layer2(h)
        finally:
            _clear_pre()
        if not gelu.used:
            _count("gelu", False, "mlp.layer2 did not take the pending input")
            out = self.layer2(self.activation(h))
        return out


# ------------------------------------------------------------------------------------------------ install
def _cosmos_module():
    import comfy.ldm.cosmos.predict2 as p2
    return p2


def install(parts=None, module=None):
    """Put the adapter on ``module``'s Block / Attention / GPT2FeedForward classes (default: ComfyUI's
    comfy.ldm.cosmos.predict2) for ``parts`` (default: WEIGHTFERRY_FUSED_BLOCK). install(()) gives ComfyUI's
    methods back. Returns the parts in effect."""
    if module is None:
        try:
            module = _cosmos_module()
        except Exception as exc:  # noqa: BLE001 -- no ComfyUI Cosmos model: nothing to patch
            log_warn(f"int8 block: ComfyUI's Cosmos model not found ({exc}); not installed.")
            return ()
    parts = tuple(p for p in (wanted_parts() if parts is None else parts) if p in PARTS)
    if "ln" in parts and "modq" not in parts:
        parts = tuple(p for p in parts if p != "ln")     # the LayerNorm travels with the pending scale-and-shift
    orig = _state.get("orig")
    if orig is None or orig.get("module") is not module:
        orig = _state["orig"] = {"module": module, "forward": module.Block.forward,
                                 "compute_qkv": module.Attention.compute_qkv,
                                 "mlp_forward": module.GPT2FeedForward.forward}
    _state["parts"] = parts
    module.Block.forward = _block_forward if parts else orig["forward"]
    module.Attention.compute_qkv = _compute_qkv if "qkv" in parts else orig["compute_qkv"]
    module.GPT2FeedForward.forward = _mlp_forward if ("gelu" in parts or "modq" in parts) else orig["mlp_forward"]
    if parts:
        log_info(f"int8 block: {', '.join(parts)} (WEIGHTFERRY_FUSED_BLOCK).")
    return parts


def uninstall():
    """ComfyUI's own methods back on the classes ``install`` patched."""
    orig = _state.get("orig")
    if orig is not None:
        install((), orig["module"])
    _state["parts"] = ()

"""Flat block layouts and block discovery of block streaming (streaming/common.py:81-151 of the reference).

A streamed block's parameters live in one flat uint8 buffer (a pinned host buffer per block, a GPU slot per slot),
each parameter at an offset aligned to _ALIGN bytes, the total rounded up to _ALIGN; one copy moves a whole block."""
import torch

_STATE_ATTR = "_weightferry_stream_state"
_ACTIVE_ATTR = "_weightferry_stream_active_owner"
_ALIGN = 256  # bytes, alignment of each parameter view inside a flat buffer

# attribute holding the transformer block list, DiT lists first (streaming/common.py:123-133)
_BLOCK_LIST_ATTRS = ("blocks", "transformer_blocks", "layers", "block")


def _nbytes(shape, dtype):
    n = 1
    for d in shape:
        n *= int(d)
    return n * dtype.itemsize


def _align_up(n, a=_ALIGN):
    return (n + a - 1) // a * a


def _flat_layout(specs):
    """Byte offsets of each (shape, dtype) spec inside one flat buffer, and the total size (aligned)."""
    offsets, offset = [], 0
    for shape, dtype in specs:
        offset = _align_up(offset)
        offsets.append(offset)
        offset += _nbytes(shape, dtype)
    return offsets, _align_up(offset)


def _views(flat, specs, offsets):
    """Typed, shaped views of each spec into the flat uint8 buffer."""
    return [flat[o:o + _nbytes(shape, dtype)].view(dtype).view(shape) for (shape, dtype), o in zip(specs, offsets)]


def _block_list_attr(dit):
    for name in _BLOCK_LIST_ATTRS:
        lst = getattr(dit, name, None)
        if isinstance(lst, torch.nn.ModuleList) and len(lst) > 0:
            return name
    return None


def _blocks(dit):
    name = _block_list_attr(dit)
    return getattr(dit, name) if name else []


def _param_owner(blk, name):
    """(module, parameter key) of the parameter ``name`` (as named_parameters() of ``blk`` gives it)."""
    mod_name, _, param_key = name.rpartition(".")
    return (blk.get_submodule(mod_name) if mod_name else blk), param_key


def _specs(blk):
    """(shape, dtype) of every parameter of a block, in parameters() order."""
    return [(tuple(p.shape), p.dtype) for p in blk.parameters()]

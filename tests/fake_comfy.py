"""Stand-ins for the host application's modules that the drop-in patches (ComfyUI-GGUF's ``ops``), registered in
sys.modules under the name the reference looks for (a module whose name ends in "ComfyUI-GGUF.ops",
enhancers/gguf_dequant.py:554). They record calls so tests can see which path ran."""
import sys
import types

import torch


class GGMLTensor(torch.Tensor):
    """A uint8 tensor of GGUF blocks carrying tensor_type / tensor_shape, like ComfyUI-GGUF's GGMLTensor."""

    @staticmethod
    def __new__(cls, data, tensor_type, tensor_shape, patches=None):
        return torch.Tensor._make_subclass(cls, data, False)

    def __init__(self, data, tensor_type, tensor_shape, patches=None):
        self.tensor_type = tensor_type
        self.tensor_shape = tensor_shape
        self.patches = patches or []

    @classmethod
    def __torch_function__(cls, func, types_, args=(), kwargs=None):
        kwargs = kwargs or {}
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)


def make_ops_module(name="custom_nodes.ComfyUI-GGUF.ops"):
    ops = types.ModuleType(name)
    ops.calls = []

    def dequantize_tensor(tensor, dtype=None, dequant_dtype=None):
        ops.calls.append(("dequantize_tensor", getattr(tensor, "tensor_type", None), dtype, dequant_dtype))
        return "host-dequant"

    class GGMLLayer:
        dequant_dtype = None
        patch_dtype = None

        def get_weight(self, tensor, dtype):
            ops.calls.append(("get_weight", getattr(tensor, "tensor_type", None), dtype))
            return "host-get-weight"

    ops.dequantize_tensor = dequantize_tensor
    ops.GGMLLayer = GGMLLayer
    ops.GGMLTensor = GGMLTensor
    sys.modules[name] = ops
    return ops


def remove_ops_module(name="custom_nodes.ComfyUI-GGUF.ops"):
    sys.modules.pop(name, None)

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


# --------------------------------------------------------------------------------------------- ModelPatcher side
class _Enum:
    def __init__(self, **kw):
        self.__dict__.update(kw)


def make_comfy_modules():
    """comfy.model_management and comfy.patcher_extension with the calls the streaming node makes: is_device_cuda,
    CallbacksMP.ON_LOAD / ON_DETACH, WrappersMP.DIFFUSION_MODEL, add_wrapper_with_key (wrappers kept per type and
    key in model_options["transformer_options"]["wrappers"], as ComfyUI keeps them)."""
    comfy = types.ModuleType("comfy")
    mm = types.ModuleType("comfy.model_management")
    pe = types.ModuleType("comfy.patcher_extension")
    mm.is_device_cuda = lambda d: torch.device(d).type == "cuda"
    pe.CallbacksMP = _Enum(ON_LOAD="on_load", ON_DETACH="on_detach")
    pe.WrappersMP = _Enum(DIFFUSION_MODEL="diffusion_model")

    def add_wrapper_with_key(wrapper_type, key, fn, options, is_model_options=False):
        to = options.setdefault("transformer_options", {}) if is_model_options else options
        to.setdefault("wrappers", {}).setdefault(wrapper_type, {}).setdefault(key, []).append(fn)
    pe.add_wrapper_with_key = add_wrapper_with_key
    comfy.model_management, comfy.patcher_extension = mm, pe
    sys.modules.update({"comfy": comfy, "comfy.model_management": mm, "comfy.patcher_extension": pe})
    return comfy


def remove_comfy_modules():
    for k in ("comfy", "comfy.model_management", "comfy.patcher_extension"):
        sys.modules.pop(k, None)


class FakeModelPatcher:
    """The parts of ComfyUI's ModelPatcher the node uses: clone (shares the model, copies options and callbacks),
    add_callback, model_options; load / detach fire the ON_LOAD / ON_DETACH callbacks; apply_model runs the diffusion
    model through the DIFFUSION_MODEL wrappers (each called as wrapper(executor, *args))."""

    def __init__(self, diffusion_model, load_device="cuda"):
        self.model = types.SimpleNamespace(diffusion_model=diffusion_model)
        self.load_device = torch.device(load_device)
        self.model_options = {"transformer_options": {}}
        self.callbacks = {}

    def clone(self):
        import copy
        c = FakeModelPatcher.__new__(FakeModelPatcher)
        c.model, c.load_device = self.model, self.load_device
        c.model_options = copy.deepcopy(self.model_options)
        c.callbacks = {k: list(v) for k, v in self.callbacks.items()}
        return c

    def add_callback(self, kind, fn):
        self.callbacks.setdefault(kind, []).append(fn)

    def load(self, device=None):
        for fn in self.callbacks.get("on_load", []):
            fn(self, device if device is not None else self.load_device, 0, False, True)

    def detach(self):
        for fn in self.callbacks.get("on_detach", []):
            fn(self, True)

    def apply_model(self, *args, **kwargs):
        fn = self.model.diffusion_model
        for key, fns in self.model_options["transformer_options"].get("wrappers", {}).get("diffusion_model", {}).items():
            for w in fns:
                fn = (lambda w_, inner: lambda *a, **k: w_(inner, *a, **k))(w, fn)
        return fn(*args, **kwargs)

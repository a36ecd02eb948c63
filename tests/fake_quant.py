"""A stand-in for ComfyUI's int8 QuantizedTensor (TensorWiseINT8Layout): a tensor whose value is the dequantised
weight (so torch.nn.functional.linear works on it, as ComfyUI's does through dispatch) carrying the int8 data, the
scale and the layout parameters the int8 path reads (_layout_cls, _qdata, _params)."""
import types

import torch


class FakeQT(torch.Tensor):
    @staticmethod
    def __new__(cls, w_q, scale, convrot=True, transposed=False, groupsize=256):
        deq = (w_q.float() * torch.as_tensor(scale, dtype=torch.float32).reshape(-1, 1)).to(torch.bfloat16)
        return torch.Tensor._make_subclass(cls, deq, False)

    def __init__(self, w_q, scale, convrot=True, transposed=False, groupsize=256):
        self._layout_cls = "TensorWiseINT8Layout"
        self._qdata = w_q
        self._params = types.SimpleNamespace(scale=scale, convrot=convrot, transposed=transposed,
                                             convrot_groupsize=groupsize)

    @classmethod
    def __torch_function__(cls, func, types_, args=(), kwargs=None):
        kwargs = kwargs or {}
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)


class Lin:
    """A ComfyUI-style linear whose forward calls self._forward(input, weight, bias)."""

    def __init__(self, weight, bias=None):
        self.weight, self.bias = weight, bias

    def _forward(self, input, weight, bias):
        return torch.nn.functional.linear(input, weight, bias)

    def __call__(self, x):
        return self._forward(x, self.weight, self.bias)

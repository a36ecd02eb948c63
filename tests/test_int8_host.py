"""Host-side behaviour of enhancers.fused_int8 on the CPU: _Overrides installs and removes the per-call _forward
and the shared-quantisation cache (enhancers/fused_int8.py:311-332 of the reference); _int8_quantised declines
every case outside the reference's eligibility (:129-147), and _shared_forward then runs
torch.nn.functional.linear and counts the fallback (:279-292); a pending input is materialised for the fallback."""
import torch

from conftest import sub
from fake_quant import FakeQT, Lin

fi = sub("enhancers.fused_int8")
fs = sub("enhancers.fused_state")


def _weight(n=16, k=256, **kw):
    g = torch.Generator().manual_seed(n + k)
    w_q = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int64).to(torch.int8)
    return FakeQT(w_q, torch.full((n,), 0.01), **kw)


def test_overrides_install_and_restore():
    lins = [Lin(_weight()), Lin(_weight())]
    special = lambda i, w, b: "special"  # noqa: E731
    with fi._Overrides([lins[0], (lins[1], special)]) as ov:
        assert lins[0].__dict__["_forward"] is fi._shared_forward
        assert lins[1].__dict__["_forward"] is special
        assert fi._tls.qkv == {} and not ov.outer
        with fi._Overrides([lins[0]]) as inner:        # already overridden: left alone; outer cache kept
            assert inner.outer and inner.layers == []
        assert fi._tls.qkv == {}
    assert "_forward" not in lins[0].__dict__ and "_forward" not in lins[1].__dict__
    assert getattr(fi._tls, "qkv", None) is None


def test_ineligible_cases_return_none():
    x = torch.randn(8, 256).to(torch.bfloat16)
    fi._tls.qkv = {}
    try:
        assert fi._int8_quantised(x, _weight(), None) is None                          # CPU input
        assert fi._int8_quantised(x, _weight(), torch.zeros(16)) is None               # bias
        assert fi._int8_quantised(x, _weight(convrot=False), None) is None             # not ConvRot
        assert fi._int8_quantised(x, _weight(transposed=True), None) is None
        assert fi._int8_quantised(x, _weight(groupsize=128), None) is None
        assert fi._int8_quantised(x, torch.zeros(16, 256), None) is None               # not a quantized weight
    finally:
        fi._tls.qkv = None
    assert fi._int8_quantised(x, _weight(), None) is None                              # outside _Overrides


def test_shared_forward_falls_back_and_counts():
    fs.stats(reset=True)
    w = _weight()
    x = torch.randn(4, 256).to(torch.bfloat16)
    lin = Lin(w)
    with fi._Overrides([lin]):
        y = lin(x)
    ref = torch.nn.functional.linear(x, w.as_subclass(torch.Tensor))
    assert torch.equal(y, ref)
    st = fs.stats()
    assert st["qkv"]["fallback"] == 1 and st["qkv"]["used"] == 0 and "FakeQT" in st["qkv"]["why"]


def test_pending_input_is_materialised_for_the_fallback():
    fs.stats(reset=True)
    w = _weight()
    x = torch.randn(4, 256).to(torch.bfloat16)
    scale, shift = torch.full((256,), 0.5).to(torch.bfloat16), torch.full((256,), 0.25).to(torch.bfloat16)
    pre = fi._set_pre(x, "mod", scale=scale, shift=shift)
    lin = Lin(w)
    with fi._Overrides([lin]):
        y = lin(x)
    fi._clear_pre()
    assert pre["used"]
    real = x * (1 + scale) + shift
    assert torch.equal(y, torch.nn.functional.linear(real, w.as_subclass(torch.Tensor)))


def test_residual_forward_without_pending_residual_is_shared_forward():
    w = _weight()
    x = torch.randn(4, 256).to(torch.bfloat16)
    fi._tls.res = None
    y = fi._residual_forward(x, w, None)
    assert torch.equal(y, torch.nn.functional.linear(x, w.as_subclass(torch.Tensor)))


def test_int8_linear_declines_cpu():
    assert fi.int8_linear(torch.randn(4, 256).to(torch.bfloat16), torch.zeros(8, 256, dtype=torch.int8),
                          torch.ones(8)) is None

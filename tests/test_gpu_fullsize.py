"""GPU parity at the full sizes of the two workloads the other GPU tests cover only in smaller pieces.

* Q8_0 dequantisation of one 5120 x 5120 weight: float32 N(0, 0.02) weights (numpy PCG64, seed 1234) encoded as
  GGUF Q8_0 (32-value blocks, d = f16(absmax / 127)), dequantised with MID float16 and float32 to bfloat16 through
  the drop-in ``dequantize`` -- every one of the 26,214,400 values bit-exact against the oracle.
* A streamed forward of 40 Wan-2.1-14B-shaped blocks with Q4_K weights (197.7 MB a block, 7.9 GB in pinned host
  memory), 4096 tokens bf16 N(0, 1) (seed 99), text context 512 tokens: block streaming with 2 GPU slots and chunk
  streaming with 96 MB chunks through 4 slots, four forwards each, every output ``torch.equal`` to the same 40
  blocks resident on the GPU (the reference's criterion for streaming, tests/test_streaming.py:222).
"""
import sys

import numpy as np
import pytest
import torch

from conftest import sub
from oracle import lib

pytestmark = pytest.mark.gpu

encode = sub("gguf_encode")


def _say(msg):
    print(msg, file=sys.stderr, flush=True)


@pytest.mark.parametrize("mid", [torch.float16, torch.float32])
def test_q8_0_5120_square_bit_exact(native, mid):
    gd = sub("enhancers.gguf_dequant")
    shape = (5120, 5120)
    raw = encode.encode(encode.weights(shape, seed=1234), 8)
    assert raw.size == 27_852_800
    _say(f"case Q8_0 5120x5120 mid={mid}")
    out = gd.dequantize(torch.from_numpy(raw).cuda(), 8, shape, mid, torch.bfloat16)
    torch.cuda.synchronize()
    assert out.shape == shape and out.dtype == torch.bfloat16
    got = out.cpu().view(torch.int16).numpy().view(np.uint16).ravel()
    ref = lib.dequant(raw, 8, {torch.float16: 0, torch.float32: 2}[mid], 1, shape[0] * shape[1])
    bad = np.nonzero(got != ref)[0]
    assert bad.size == 0, (bad[:8], got[bad[:8]], ref[bad[:8]])


@pytest.fixture(scope="module")
def wan40():
    """The 40-block Q4_K stack on the CPU, its inputs on the GPU, and its resident output."""
    syn = sub("streaming.synthetic")
    _say("case wan40: building 40 Q4_K blocks (seed 1234)")
    model = syn.WanLikeStack(n_blocks=40, qtype=12, mode="auto")
    model.fill_random(1234)
    g = torch.Generator().manual_seed(99)
    x = torch.randn((1, 4096, 5120), generator=g).to(torch.bfloat16).cuda()
    ctx = torch.randn((1, 512, 5120), generator=g).to(torch.bfloat16).cuda()
    _say("case wan40: resident forward")
    model.cuda()
    with torch.no_grad():
        ref = model(x, ctx)
    torch.cuda.synchronize()
    model.cpu()
    torch.cuda.empty_cache()
    yield model, x, ctx, ref
    del model
    torch.cuda.empty_cache()


def _forwards_equal(sm, x, ctx, ref, n, what):
    for i in range(n):
        with torch.no_grad():
            y = sm(x, ctx)
        torch.cuda.synchronize()
        _say(f"case wan40 {what}: forward {i} done")
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"{what}: forward {i} differs"


@pytest.mark.timeout(600)
def test_wan40_block_streaming_equals_resident(native, wan40):
    dn = sub("streaming.dit_node")
    model, x, ctx, ref = wan40
    _say("case wan40 block streaming: capture")
    sm = dn.apply_streaming(model, device="cuda", prefetch_slots=2, profile=False)
    try:
        assert sm.state.num_slots == 2 and sm.state.flat_bytes == 197_710_848
        _forwards_equal(sm, x, ctx, ref, 4, "block streaming")
    finally:
        sm.teardown(device="cpu")
    torch.cuda.empty_cache()


@pytest.mark.timeout(600)
def test_wan40_chunk_streaming_equals_resident(native, wan40):
    dn = sub("streaming.dit_node")
    model, x, ctx, ref = wan40
    _say("case wan40 chunk streaming: capture")
    sm = dn.apply_streaming(model, device="cuda", chunk=True, chunk_bytes=96 * 1024 ** 2, chunk_slots=4)
    try:
        _forwards_equal(sm, x, ctx, ref, 4, "chunk streaming")     # forward 0 learns the order, 1..3 stream chunks
        assert sm.state.n_types == 3 and not sm.state.calibrating
    finally:
        sm.teardown(device="cpu")
    torch.cuda.empty_cache()

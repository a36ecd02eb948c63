"""A synthetic stack of Wan-2.1-14B-shaped DiT blocks with GGUF weights, for benchmarks and tests of block
streaming: dim 5120, 40 heads of 128, FFN 13824, text context of 512 tokens. Per block: self-attention (q, k, v, o),
cross-attention (q, o on the tokens, k, v on the context), FFN (up, GELU-tanh, down), each linear a GGUFLinear with
a bias, LayerNorms without parameters before each part -- 351,272,960 weights, 197,591,040 bytes in Q4_K. Weights
are random blocks (random quants and scale codes, f16 scales of a fixed small magnitude), which is all a
throughput measurement needs; different seeds give different blocks."""
import numpy as np
import torch

from ..enhancers.fused_gguf import GGUFLinear

_F16_FIELDS = {12: (0, 2), 13: (0, 2), 14: (208,)}
_TS = {12: 144, 13: 176, 14: 210}


def random_gguf_bytes(n_out, n_in, qtype, seed, d=2.0e-5, dmin=4.0e-5):
    """Random blocks of GGML type qtype for an [n_out, n_in] weight with the f16 scale fields set to d / dmin."""
    ts = _TS[qtype]
    nb = n_out * n_in // 256
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=nb * ts, dtype=np.uint8).reshape(nb, ts)
    vals = [d, dmin]
    for off, v in zip(_F16_FIELDS[qtype], vals):
        raw[:, off:off + 2] = np.array([v], dtype=np.float16).view(np.uint8)
    return torch.from_numpy(raw.reshape(-1))


class WanLikeBlock(torch.nn.Module):
    def __init__(self, dim=5120, heads=40, ffn=13824, qtype=12, mode="auto"):
        super().__init__()
        self.dim, self.heads = dim, heads
        L = lambda i, o: GGUFLinear(i, o, qtype, bias=True, mode=mode)  # noqa: E731
        self.q, self.k, self.v, self.o = L(dim, dim), L(dim, dim), L(dim, dim), L(dim, dim)
        self.cq, self.ck, self.cv, self.co = L(dim, dim), L(dim, dim), L(dim, dim), L(dim, dim)
        self.up, self.down = L(dim, ffn), L(ffn, dim)

    def linears(self):
        return [self.q, self.k, self.v, self.o, self.cq, self.ck, self.cv, self.co, self.up, self.down]

    def fill_random(self, seed):
        for i, lin in enumerate(self.linears()):
            lin.weight.data.copy_(random_gguf_bytes(lin.out_features, lin.in_features, lin.qtype, seed * 100 + i))
            g = torch.Generator().manual_seed(seed * 100 + i)
            lin.bias.data.copy_((torch.randn(lin.out_features, generator=g) * 0.01).to(torch.bfloat16))

    def _attn(self, q, k, v):
        B, T, D = q.shape
        S = k.shape[1]
        h, hd = self.heads, D // self.heads
        q = q.view(B, T, h, hd).transpose(1, 2)
        k = k.view(B, S, h, hd).transpose(1, 2)
        v = v.view(B, S, h, hd).transpose(1, 2)
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v)
        return o.transpose(1, 2).reshape(B, T, D)

    def forward(self, x, ctx):
        D = self.dim
        h = torch.nn.functional.layer_norm(x, (D,))
        x = x + self.o(self._attn(self.q(h), self.k(h), self.v(h)))
        h = torch.nn.functional.layer_norm(x, (D,))
        x = x + self.co(self._attn(self.cq(h), self.ck(ctx), self.cv(ctx)))
        h = torch.nn.functional.layer_norm(x, (D,))
        return x + self.down(torch.nn.functional.gelu(self.up(h), approximate="tanh"))


def gguf_tensors(model, attr="blocks"):
    """(name, GGML type, torch shape, bytes) of every parameter of the stack's blocks in parameters() order, named
    "<attr>.<block index>.<parameter name>": GGUFLinear weights as their quantised blocks, bf16 biases as BF16."""
    out = []
    for i, blk in enumerate(getattr(model, attr)):
        for mname, mod in blk.named_modules():
            if not isinstance(mod, GGUFLinear):
                continue
            out.append((f"{attr}.{i}.{mname}.weight", mod.qtype, (mod.out_features, mod.in_features), mod.weight.data))
            if mod.bias is not None:
                out.append((f"{attr}.{i}.{mname}.bias", 30, (mod.out_features,), mod.bias.data))
    return out


def write_gguf_model(model, path, alignment=256):
    """The stack's block parameters as a GGUF file (general.architecture "wan"), tensors in parameters() order at
    ``alignment``: with the flat layout's 256-byte alignment a block is one contiguous range of the file."""
    from ..core.tiers.gguf_file import write_gguf
    return write_gguf(path, gguf_tensors(model), {"general.architecture": "wan"}, alignment=alignment)


class WanLikeStack(torch.nn.Module):
    def __init__(self, n_blocks=40, dim=5120, heads=40, ffn=13824, qtype=12, mode="auto"):
        super().__init__()
        self.blocks = torch.nn.ModuleList(WanLikeBlock(dim, heads, ffn, qtype, mode) for _ in range(n_blocks))

    def fill_random(self, seed=1234):
        for i, b in enumerate(self.blocks):
            b.fill_random(seed + i)

    def forward(self, x, ctx):
        for b in self.blocks:
            x = b(x, ctx)
        return x

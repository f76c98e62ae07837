"""The step programs of a decoder-only transformer, as an engine writes them
with the program builder: token embedding, per layer RMSNorm → q/k/v →
RoPE → KV stores into ring caches → attention (GQA) → output projection →
residual, RMSNorm → gate/up → SiLU·up → down → residual, then the final norm,
the unembedding and the greedy token.

Sources are named per layer (``l{i}_q_proj``, ``l{i}_k_cache``, ...); the
engine binds them by name.  Weights are ``out_in`` ([outputs, inputs]).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

from .build import ProgramBuilder, program
from .graph import BF16, CACHE_F16, F16, F32, GELU_TANH, SILU, AttnSpec, Paged, Program, Ring, RopeSpec, whole_row


@dataclass(frozen=True)
class DecoderDims:
    d_model: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    context: int          # positions a ring cache holds (a sequence's length bound)
    rope_theta: float = 10000.0
    eps: float = 1e-5
    weight_type: str = F16
    cache_elem: str = CACHE_F16
    slots: int = 1        # sequences the caches hold
    act: str = SILU       # the gated MLP's activation: SILU or GELU_TANH
    embed_factor: float = 1.0  # the gathered embedding row's scale (Gather's factor, Eval.hs:528-535)

    @property
    def q_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_width(self) -> int:
        return self.kv_heads * self.head_dim

    def layer_params(self) -> int:
        d, f = self.d_model, self.ffn
        return d * self.q_width + 2 * d * self.kv_width + self.q_width * d + 3 * d * f + 2 * d

    def params(self) -> int:
        return self.layers * self.layer_params() + 2 * self.vocab * self.d_model + self.d_model


# The configurations: the tiny f32 decode and the 1B-class f16 decode.
TINY = DecoderDims(d_model=64, layers=2, heads=4, kv_heads=4, head_dim=16, ffn=256, vocab=256, context=16,
                   weight_type=F32)
# The tiny decode with grouped queries (4 heads over 2 kv heads) and a ring of
# 256 positions, so that attention at a position past 127 runs in two splits.
TINY_GQA = DecoderDims(d_model=64, layers=2, heads=4, kv_heads=2, head_dim=16, ffn=256, vocab=256, context=256,
                       weight_type=F32)
# The tiny decode with bf16 weights (the reference builder's type) and a
# GELU-tanh gated MLP (the reference's activation).
TINY_GELU_BF16 = DecoderDims(d_model=64, layers=2, heads=4, kv_heads=2, head_dim=16, ffn=256, vocab=256, context=32,
                             weight_type=BF16, act=GELU_TANH)
ONE_B = DecoderDims(d_model=2048, layers=16, heads=32, kv_heads=8, head_dim=64, ffn=8192, vocab=32000, context=4096)
# The 1B prefill: four sequences of 2048 rows into a ring of 4096 positions.
ONE_B_PREFILL = DecoderDims(d_model=2048, layers=16, heads=32, kv_heads=8, head_dim=64, ffn=8192, vocab=32000,
                            context=4096, slots=4)
# The tiny decode with its embedding row scaled as the reference's embedding
# program scales it (ProgramTest.hs:785-789: factor 5.65625), the ring of 32.
TINY_EMBED = DecoderDims(d_model=64, layers=2, heads=4, kv_heads=4, head_dim=16, ffn=256, vocab=256, context=32,
                         weight_type=F32, embed_factor=5.65625)
# A small f16 decoder the prefill kernels take whole (anchors of 256 rows,
# heads of 64, two kv heads to a group), for checking prefill against the
# f64 evaluator.
SMALL_PREFILL = DecoderDims(d_model=256, layers=2, heads=8, kv_heads=4, head_dim=64, ffn=512, vocab=512, context=256,
                            slots=2)


def decoder_step(dims: DecoderDims, name: str = "decode", embed: bool = True,
                 layers: Optional[int] = None, position_bound: Optional[int] = None,
                 rope_rotated: Optional[int] = None, paging: Optional[tuple] = None) -> Program:
    """One step of the decoder over the rows it is given (one a decode step,
    a sequence's run of rows a prefill): ``embed`` gathers each token's row
    of ``embed`` (else the rows ``x`` are an input); outputs ``logits`` and
    the greedy ``token`` of every row.  Positions are declared below
    ``position_bound`` (default: the context), which decides whether a
    step's KV stores fit the ring in place (Plan.hs:276-281).  RoPE turns
    ``rope_rotated`` pairs of each head (default: all, head_dim / 2).
    ``paging`` = (block size, pool blocks): the caches are paged pools
    (Graph.hs:144-152) and each row carries its block table (``blocks``, the
    context's positions in blocks) in place of its ring slot."""
    L = dims.layers if layers is None else layers
    wt = dims.weight_type

    def body(b: ProgramBuilder):
        pos = b.row_ints("position", 1, dims.context if position_bound is None else position_bound)
        if paging is None:
            slot = b.row_ints("slot", 1, dims.slots)
            layout = Ring(dims.slots, dims.kv_heads, dims.context, dims.head_dim)
        else:
            block_size, pool_blocks = paging
            slot = b.row_ints("blocks", dims.context // block_size, pool_blocks)
            layout = Paged(pool_blocks, block_size, dims.kv_heads, dims.head_dim)
        if embed:
            tokens = b.row_ints("tokens", 1, dims.vocab)
            table = b.weight("embed", [dims.vocab, dims.d_model], wt)
            x = b.gather("x0", table, tokens, dims.embed_factor)
        else:
            x = b.input("x", whole_row(dims.d_model), F32)
        rope = RopeSpec(dims.rope_theta, dims.head_dim // 2 if rope_rotated is None else rope_rotated)
        attn = AttnSpec(dims.heads, dims.kv_heads, dims.head_dim, None, 1.0 / math.sqrt(dims.head_dim))
        for i in range(L):
            p = f"l{i}_"
            g_attn = b.weight(p + "attn_norm", [dims.d_model], F32)
            wq = b.weight(p + "q_proj", [dims.q_width, dims.d_model], wt)
            wk = b.weight(p + "k_proj", [dims.kv_width, dims.d_model], wt)
            wv = b.weight(p + "v_proj", [dims.kv_width, dims.d_model], wt)
            wo = b.weight(p + "o_proj", [dims.d_model, dims.q_width], wt)
            g_mlp = b.weight(p + "mlp_norm", [dims.d_model], F32)
            wg = b.weight(p + "gate_proj", [dims.ffn, dims.d_model], wt)
            wu = b.weight(p + "up_proj", [dims.ffn, dims.d_model], wt)
            wd = b.weight(p + "down_proj", [dims.d_model, dims.ffn], wt)
            kc = b.cache(p + "k_cache", layout, dims.cache_elem)
            vc = b.cache(p + "v_cache", layout, dims.cache_elem)
            a = b.rmsnorm(p + "attn_in", dims.eps, g_attn, 1.0, x)
            q = b.linear(p + "q", wq, dims.head_dim, a)
            k = b.linear(p + "k", wk, dims.head_dim, a)
            v = b.linear(p + "v", wv, dims.head_dim, a)
            qr = b.rope(p + "q_rot", rope, pos, q)
            kr = b.rope(p + "k_rot", rope, pos, k)
            b.kv_store(p + "store_k", kc, pos, slot, kr)
            b.kv_store(p + "store_v", vc, pos, slot, v)
            o = b.attend(p + "attn", attn, qr, kc, vc, pos, slot)
            out = b.linear(p + "o", wo, 0, o)
            x1 = b.add(p + "x1", x, out)
            m = b.rmsnorm(p + "mlp_in", dims.eps, g_mlp, 1.0, x1)
            gate = b.linear(p + "gate", wg, 0, m)
            up = b.linear(p + "up", wu, 0, m)
            act = b.gelu_mul(p + "act", gate, up, dims.act)
            down = b.linear(p + "down", wd, 0, act)
            x = b.add(p + "x2", x1, down)
        g_final = b.weight("final_norm", [dims.d_model], F32)
        head = b.weight("lm_head", [dims.vocab, dims.d_model], wt)
        n = b.rmsnorm("final_normed", dims.eps, g_final, 1.0, x)
        logits = b.linear("logits", head, 0, n)
        b.output("logits", logits)
        b.output("token", b.argmax("token", logits))

    return program(name, body)

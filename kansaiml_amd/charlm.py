"""Config C4: the quantized decoder-only char-LM forward on the HIP backend.

The architecture is the reference's BigGPT
(examples/tinyshakespeare/train_shakespeare_large.py:61-79) built from its
nn modules (python/kansai/nn.py): token + learned position embedding,
N pre-LN TransformerBlocks (nn.py:430-478: x + attn(LN1 x), then
x + fc2(GELU(fc1(LN2 x)))) under one causal mask, a final LayerNorm and the
vocabulary head.  As in BigGPT.forward (:86), the mask applies when the
sequence fills the position table (seq == block size); a shorter sequence
attends over all of its keys.  MultiHeadAttention (nn.py:334-427) has no projection bias;
the FFN Linears and the head do.

Every Linear is int8 here: weights quantized once per output channel
(packed [out, in]), activations quantized per tensor on the fly, int32
accumulation, dequantize + bias in the GEMM epilogue.  Q, K and V share one
GEMM (their weights concatenated to [D, 3D]; with per-channel weight scales
this is the same arithmetic as three GEMMs).  Softmax, LayerNorm, GELU and
the residual adds are fp32.  The forward is traced once into a KIR graph,
fused, and replayed with run_hip_planned.
"""

from __future__ import annotations

import math

import numpy as np

from . import kir
from .device import DeviceTensor
from .quantize import QTensor


# Parameter names of the reference's BigGPT, in its named_parameters() order
# (train_shakespeare_large.py:61-79 over nn.py:19-39: tok_embed, pos_embed,
# blocks.i = TransformerBlock nn.py:466-472 {ln1, attn (w_q, w_k, w_v, w_o,
# nn.py:384-390), ln2, fc1, fc2}, ln_f, head), with the key each has here.
_BLOCK_PARAMS = (("ln1.weight", "ln1_w"), ("ln1.bias", "ln1_b"), ("attn.w_q", "w_q"), ("attn.w_k", "w_k"),
                 ("attn.w_v", "w_v"), ("attn.w_o", "w_o"), ("ln2.weight", "ln2_w"), ("ln2.bias", "ln2_b"),
                 ("fc1.weight", "fc1_w"), ("fc1.bias", "fc1_b"), ("fc2.weight", "fc2_w"), ("fc2.bias", "fc2_b"))


class CharLMWeights:
    """fp32 parameters of the model, host side (numpy), seeded.

    named_parameters() / set_parameter() use the reference BigGPT's names, so
    kansaiml_amd.serialize reads and writes checkpoints of it."""

    def __init__(self, vocab=65, d_model=384, heads=6, layers=6, d_ff=1536, seq=256, seed=0, std=0.02,
                 bias_std=0.0):
        g = np.random.Generator(np.random.PCG64(seed))
        f32 = np.float32
        self.vocab, self.d_model, self.heads, self.layers, self.d_ff, self.seq = vocab, d_model, heads, layers, d_ff, seq
        # nn.Embedding: std 1/sqrt(embed_dim) (nn.py:637-641)
        self.tok = (g.standard_normal((vocab, d_model)) / math.sqrt(d_model)).astype(f32)
        self.pos = (g.standard_normal((seq, d_model)) / math.sqrt(d_model)).astype(f32)

        def lin(i, o):
            return (g.standard_normal((i, o)) * std).astype(f32)

        def bias(o):
            return (g.standard_normal(o) * bias_std).astype(f32) if bias_std else np.zeros(o, f32)

        self.blocks = []
        for _ in range(layers):
            self.blocks.append(dict(
                ln1_w=np.ones(d_model, f32), ln1_b=np.zeros(d_model, f32),
                w_q=lin(d_model, d_model), w_k=lin(d_model, d_model), w_v=lin(d_model, d_model),
                w_o=lin(d_model, d_model),
                ln2_w=np.ones(d_model, f32), ln2_b=np.zeros(d_model, f32),
                fc1_w=lin(d_model, d_ff), fc1_b=bias(d_ff), fc2_w=lin(d_ff, d_model), fc2_b=bias(d_model)))
        self.lnf_w, self.lnf_b = np.ones(d_model, f32), np.zeros(d_model, f32)
        self.head_w, self.head_b = lin(d_model, vocab), bias(vocab)

    def _slots(self):
        """(reference name, container, key) for every parameter."""
        yield "tok_embed.weight", self, "tok"
        yield "pos_embed.weight", self, "pos"
        for i, b in enumerate(self.blocks):
            for name, key in _BLOCK_PARAMS:
                yield f"blocks.{i}.{name}", b, key
        for name, key in (("ln_f.weight", "lnf_w"), ("ln_f.bias", "lnf_b"), ("head.weight", "head_w"),
                          ("head.bias", "head_b")):
            yield name, self, key

    def named_parameters(self):
        for name, c, key in self._slots():
            yield name, (c[key] if isinstance(c, dict) else getattr(c, key))

    def set_parameter(self, name: str, value) -> None:
        """Stores a loaded value (an int8 QTensor is dequantized on the device
        first, quantize.py:73-77)."""
        from .quantize import QTensor
        for n, c, key in self._slots():
            if n == name:
                if isinstance(value, QTensor):
                    value = value.dequantize().numpy()
                arr = np.array(value, dtype=np.float32)
                if isinstance(c, dict):
                    c[key] = arr
                else:
                    setattr(c, key, arr)
                return
        raise KeyError(name)


class CharLM:
    """Device-resident int8 model; `forward(ids)` returns fp32 logits
    [batch * seq, vocab] (numpy by default).

    named_parameters() yields the device parameters under the reference
    BigGPT's names (Q, K and V as row slices of the fused QKV weight), so
    kansaiml_amd.serialize saves an int8 checkpoint of the model and loads
    one (or a float32 checkpoint, quantized per output channel on the way)
    into it in place.  `w` stays the construction-time weights."""

    def __init__(self, w: CharLMWeights, producer_quant: bool | str = "layer_norm", act_granularity: str = "tensor",
                 qload: bool = True):
        """producer_quant (kir.quant_fusion's option): "layer_norm" (the
        default) -- each LayerNorm emits its int8 codes directly instead of
        fp32 (two passes over its input; the fastest on MI355X), and with
        per-token scales fc1 (-> GELU) quantizes its own rows inside the GEMM
        (kh_gemm_i8_quant_rows, one pass); True -- fc1's per-tensor quantize
        as well (two passes over the GEMM: less memory, slower); False --
        none.
        qload (kir.quant_fusion's option; on by default, bit-identical
        either way): the attention output's quantize runs inside the O GEMM
        that consumes it, so its codes are never written -- per tensor from
        the attention's absmax partials (kh_gemm_i8_qload), per row from its
        per-(row, head) partials (kh_gemm_i8_qload_rows).  fc1's per-tensor
        quantize stays a separate launch: quantizing on load in fc2 (K =
        1536) measured no faster.  Replayed C4 forwards on one box: per tensor
        1.1075 -> 1.1055 ms, per row 1.092 -> 1.063 ms.
        act_granularity: "tensor" (the reference's quantize_symmetric over the
        whole activation, the C4 configuration) or "row" (one scale per token;
        a LayerNorm then emits codes and scales in one pass)."""
        if act_granularity not in ("tensor", "row"):
            raise ValueError(f"act_granularity must be 'tensor' or 'row', not {act_granularity!r}")
        self.w = w
        self.producer_quant = producer_quant
        self.act_granularity = act_granularity
        self.qload = qload
        up = DeviceTensor.from_host
        self.tok, self.pos = up(w.tok), up(w.pos)
        self.blocks = []
        for b in w.blocks:
            self.blocks.append(dict(
                ln1_w=up(b["ln1_w"]), ln1_b=up(b["ln1_b"]),
                w_qkv=QTensor.from_weight(np.concatenate([b["w_q"], b["w_k"], b["w_v"]], axis=1), "col"),
                w_o=QTensor.from_weight(b["w_o"], "col"),
                ln2_w=up(b["ln2_w"]), ln2_b=up(b["ln2_b"]),
                fc1=QTensor.from_weight(b["fc1_w"], "col"), fc1_b=up(b["fc1_b"]),
                fc2=QTensor.from_weight(b["fc2_w"], "col"), fc2_b=up(b["fc2_b"])))
        self.lnf_w, self.lnf_b = up(w.lnf_w), up(w.lnf_b)
        self.head, self.head_b = QTensor.from_weight(w.head_w, "col"), up(w.head_b)
        self._graphs = {}

    def named_parameters(self):
        yield "tok_embed.weight", self.tok
        yield "pos_embed.weight", self.pos
        d = self.w.d_model
        for i, p in enumerate(self.blocks):
            qkv = p["w_qkv"]
            views = {}
            for j, key in enumerate(("w_q", "w_k", "w_v")):
                views[key] = QTensor(qkv.codes.view(j * d * d, [d, d]), qkv.scales.view(j * d, [d]), [d, d], "col",
                                     packed=True, owned=False)
            own = dict(ln1_w=p["ln1_w"], ln1_b=p["ln1_b"], w_o=p["w_o"], ln2_w=p["ln2_w"], ln2_b=p["ln2_b"],
                       fc1_w=p["fc1"], fc1_b=p["fc1_b"], fc2_w=p["fc2"], fc2_b=p["fc2_b"], **views)
            for name, key in _BLOCK_PARAMS:
                yield f"blocks.{i}.{name}", own[key]
        yield "ln_f.weight", self.lnf_w
        yield "ln_f.bias", self.lnf_b
        yield "head.weight", self.head
        yield "head.bias", self.head_b

    def set_parameter(self, name: str, value) -> None:
        from .serialize import assign_in_place
        for n, target in self.named_parameters():
            if n == name:
                return assign_in_place(name, target, value)
        raise KeyError(name)

    def _fn(self, batch, seq):
        def linear(x, qw, b=None):
            y = x.quantize(self.act_granularity).int8_matmul(qw).dequantize()
            return y.add(b) if b is not None else y

        def fn(ids):
            x = ids.embedding(self.tok, self.pos)
            for p in self.blocks:
                h = x.layer_norm(p["ln1_w"], p["ln1_b"])
                a = linear(h, p["w_qkv"]).attention(batch, seq, self.w.heads, causal=seq == self.w.seq)
                x = x.add(linear(a, p["w_o"]))
                h = x.layer_norm(p["ln2_w"], p["ln2_b"])
                x = x.add(linear(linear(h, p["fc1"], p["fc1_b"]).gelu(), p["fc2"], p["fc2_b"]))
            x = x.layer_norm(self.lnf_w, self.lnf_b)
            return linear(x, self.head, self.head_b)

        return fn

    def graph(self, batch, seq):
        key = (batch, seq)
        if key not in self._graphs:
            g = kir.quant_fusion(kir.trace(self._fn(batch, seq), np.zeros((batch, seq), np.int32)),
                                 producer_quant=self.producer_quant, qload=self.qload)
            self._graphs[key] = (g, kir.plan_memory(g))
        return self._graphs[key]

    def forward(self, ids, to_host: bool = True, observe=None):
        ids = np.asarray(ids, np.int32) if not isinstance(ids, DeviceTensor) else ids
        batch, seq = ids.shape
        if seq > self.w.seq:
            raise ValueError(f"sequence length {seq} exceeds the position table ({self.w.seq})")
        g, plan = self.graph(batch, seq)
        return kir.run_hip_planned(g, plan, None, ids, to_host=to_host, observe=observe)

    __call__ = forward

    def capture(self, batch: int, seq: int) -> "kir.HipGraph":
        """The forward for [batch, seq] token ids recorded as a HIP graph:
        g(ids, to_host=True) replays it on new ids with one launch (the
        returned device logits, with to_host=False, are overwritten by the
        next replay).  The graph reads this model's device weights in place;
        set_parameter and checkpoint loads overwrite those same buffers, so
        the next replay sees the loaded values."""
        if seq > self.w.seq:
            raise ValueError(f"sequence length {seq} exceeds the position table ({self.w.seq})")
        g, plan = self.graph(batch, seq)
        return kir.capture_hip_planned(g, plan, DeviceTensor.from_host(np.zeros((batch, seq), np.int32)))


def int8_linear_ops(w: CharLMWeights, batch: int, seq: int) -> float:
    """Integer ops (2*M*N*K) of the model's int8 Linear layers per forward."""
    m = batch * seq
    d, f = w.d_model, w.d_ff
    per_block = 2 * m * d * (3 * d) + 2 * m * d * d + 2 * m * d * f + 2 * m * f * d
    return w.layers * per_block + 2 * m * d * w.vocab


def attention_flops(w: CharLMWeights, batch: int, seq: int) -> float:
    """fp32 flops of QK^T and PV per forward, counted as full squares
    (2 * 2 * batch * heads * seq^2 * dk per layer; the causal kernel skips the
    masked half)."""
    dk = w.d_model // w.heads
    return w.layers * 2 * 2 * batch * w.heads * seq * seq * dk

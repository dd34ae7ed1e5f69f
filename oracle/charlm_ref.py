"""CPU restatement of the config-C4 forward (TEST INFRASTRUCTURE ONLY).

The reference's BigGPT (examples/tinyshakespeare/train_shakespeare_large.py:
61-79) over its nn modules (python/kansai/nn.py): Embedding (624-646),
LayerNorm (308-331: biased variance, eps 1e-5, centered / sqrt(var + eps) *
w + b), MultiHeadAttention (381-427: no projection bias, scores * 1/sqrt(d_k)
+ additive causal mask of -1e9 above the diagonal, softmax by max-subtract
(core/src/Tensor.cpp:906-913), merged heads @ w_o), TransformerBlock
(466-478: pre-LN, two residual adds; BigGPT passes the mask only when the
sequence fills the position table, :86), exact-erf GELU
(backend/cpu/src/Ops.cpp:250-256).

Every Linear goes through the oracle's int8 path (per-tensor activation
quantize, per-output-channel weight quantize, exact int32 GEMM, binary64
epilogue) so the int8 arithmetic is the C restatement's; the fp32 parts are
numpy float32.  `quantized=False` gives the plain fp32 model (x @ W + b).

Pinned on the CPU by tests/test_charlm_oracle.py: the reference tests' known
answers, closed forms, binary64 brute force of attention and of the whole
forward, causality invariants and planted mutants.
"""

from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

from . import oracle as O

f32 = np.float32


def layer_norm(x, w, b, eps=1e-5):
    mean = x.mean(axis=-1, keepdims=True, dtype=f32)
    c = (x - mean).astype(f32)
    var = (c * c).mean(axis=-1, keepdims=True, dtype=f32)
    return (c / np.sqrt(var + f32(eps)) * w + b).astype(f32)


def gelu(x):
    return (x * (f32(0.5) * (f32(1.0) + erf(x * f32(0.70710678118654752440)).astype(f32)))).astype(f32)


def attention(qkv, batch, seq, heads, causal=True, mask=None):
    """mask (optional): additive, broadcast to [batch, heads, seq, seq] and
    added to the scaled scores (nn.py:421-422), on top of the causal mask."""
    D = qkv.shape[1] // 3
    dk = D // heads
    q = qkv[:, :D].reshape(batch, seq, heads, dk).transpose(0, 2, 1, 3)
    k = qkv[:, D:2 * D].reshape(batch, seq, heads, dk).transpose(0, 2, 1, 3)
    v = qkv[:, 2 * D:].reshape(batch, seq, heads, dk).transpose(0, 2, 1, 3)
    scale = f32(1.0 / math.sqrt(dk))
    s = (q @ k.transpose(0, 1, 3, 2)).astype(f32) * scale
    if mask is not None:
        s = (s + np.asarray(mask, s.dtype)).astype(s.dtype)
    if causal:
        cm = np.where(np.arange(seq)[None, :] <= np.arange(seq)[:, None], f32(0.0), f32(-1e9))
        s = (s + cm).astype(f32)
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s).astype(f32)
    p = (e / e.sum(axis=-1, keepdims=True, dtype=f32)).astype(f32)
    o = (p @ v).astype(f32)
    return o.transpose(0, 2, 1, 3).reshape(batch * seq, D)


def causal_attention(qkv, batch, seq, heads):
    return attention(qkv, batch, seq, heads, causal=True)


def linear(x, w, b=None, quantized=True, act_granularity="tensor"):
    if not quantized:
        y = (x @ w).astype(f32)
        return y + b if b is not None else y
    if act_granularity == "row":
        qx, sx = O.ko_quantize_rows(x)
    else:
        qx, sx = O.ko_quantize_tensor(x)
        sx = [sx]
    qw, sw = O.ko_quantize_cols_packed(w)
    acc = O.ko_gemm_i8(qx, qw)
    return O.ko_epilogue(acc, sx, sw, b)


def forward(w, ids, quantized=True, act_granularity="tensor"):
    """w: kansaiml_amd.charlm.CharLMWeights (plain numpy arrays); ids [B, T]."""
    ids = np.asarray(ids)
    batch, seq = ids.shape
    x = (w.tok[ids.reshape(-1)] + np.tile(w.pos[:seq], (batch, 1))).astype(f32)
    for p in w.blocks:
        h = layer_norm(x, p["ln1_w"], p["ln1_b"])
        qkv = linear(h, np.concatenate([p["w_q"], p["w_k"], p["w_v"]], axis=1), None, quantized, act_granularity)
        # BigGPT adds its causal mask only at seq == BLOCK_SIZE
        # (train_shakespeare_large.py:86)
        a = attention(qkv, batch, seq, w.heads, causal=seq == w.seq)
        x = (x + linear(a, p["w_o"], None, quantized, act_granularity)).astype(f32)
        h = layer_norm(x, p["ln2_w"], p["ln2_b"])
        f = gelu(linear(h, p["fc1_w"], p["fc1_b"], quantized, act_granularity))
        x = (x + linear(f, p["fc2_w"], p["fc2_b"], quantized, act_granularity)).astype(f32)
    x = layer_norm(x, w.lnf_w, w.lnf_b)
    return linear(x, w.head_w, w.head_b, quantized, act_granularity)

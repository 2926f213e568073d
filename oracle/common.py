"""Oracle: shared elementwise / normalisation / attention pieces (CPU, fp32 or fp64).

Every function computes in the dtype of its input (callers pass fp32 for the
oracle proper and fp64 for pinning tests) and on its input's device.
"""
import math

import torch
import torch.nn.functional as F


def linear(x, w, b=None):
    """nn.Linear: x @ w.T + b (weights in [out, in] layout)."""
    y = x @ w.t()
    if b is not None:
        y = y + b
    return y


def layer_norm(x, eps=1e-6, weight=None, bias=None):
    """FP32LayerNorm / nn.LayerNorm over the last dim (biased variance).

    Wan norm1/norm3 (no affine) and norm2 (affine): workers/ditserve/models/wan/block.py:283,288,291.
    SD3.5 norms: workers/ditserve/models/sd35_batch.py:350,392,700,704.
    """
    mean = x.mean(-1, keepdim=True)
    var = ((x - mean) ** 2).mean(-1, keepdim=True)
    y = (x - mean) * torch.rsqrt(var + eps)
    if weight is not None:
        y = y * weight
    if bias is not None:
        y = y + bias
    return y


def rms_norm(x, weight=None, eps=1e-6):
    """RMSNorm over the last dim: x * rsqrt(mean(x^2) + eps) * weight.

    Wan: across all heads (norm_q/norm_k over D), workers/xfuser/model_executor/models/
    transformers/transformer_wan.py:165-166.  SD3.5: per head (Dh), sd35_batch.py:428-431,438-441.
    """
    y = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    if weight is not None:
        y = y * weight
    return y


def gelu_tanh(x):
    """GELU with the tanh approximation (diffusers FeedForward "gelu-approximate")."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)))


def silu(x):
    return x * torch.sigmoid(x)


def timestep_embedding(t, dim=256, flip_sin_to_cos=True, downscale_freq_shift=0.0, max_period=10000.0):
    """diffusers Timesteps(dim, flip_sin_to_cos=True, shift=0): sinusoidal embedding.

    Used by the Wan condition embedder (transformer_wan.py:331-333 -> condition_embedder)
    and the SD3.5 time_text_embed (sd35_batch.py:642-644).  Returns [N, dim] fp32.
    """
    t = torch.as_tensor(t, dtype=torch.float32)
    device = t.device                 # computed on the CPU, returned on t's device
    t = t.cpu().reshape(-1)
    half = dim // 2
    exponent = -math.log(max_period) * torch.arange(half, dtype=torch.float32) / (half - downscale_freq_shift)
    freqs = torch.exp(exponent)
    args = t[:, None].float() * freqs[None, :]
    emb = torch.cat([torch.sin(args), torch.cos(args)], dim=-1)
    if flip_sin_to_cos:
        emb = torch.cat([emb[:, half:], emb[:, :half]], dim=-1)
    return emb.to(device)


def sdpa(q, k, v, chunk=4096):
    """Non-causal softmax(q k^T / sqrt(d)) v, no mask, no dropout.

    Layout [H, Sq, D] x [H, Sk, D].  Reference semantics: the SDPA backends at
    workers/xfuser/core/attention/backends/sdpa/kernel.py:17-56 called by
    workers/xfuser/model_executor/layers/usp.py:815-824,875-908.  Queries are
    processed in chunks so S x S scores are never materialised whole.
    """
    scale = 1.0 / math.sqrt(q.shape[-1])
    out = torch.empty(q.shape[:-1] + (v.shape[-1],), dtype=q.dtype, device=q.device)
    for s0 in range(0, q.shape[-2], chunk):
        qs = q[..., s0:s0 + chunk, :]
        scores = (qs @ k.transpose(-1, -2)) * scale
        out[..., s0:s0 + chunk, :] = torch.softmax(scores, dim=-1) @ v
    return out


def sdpa_lse(q, k, v):
    """Like sdpa() but also returns the natural-log sum-exp of the scaled scores, [H, Sq]."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    scores = (q @ k.transpose(-1, -2)) * scale
    return torch.softmax(scores, dim=-1) @ v, torch.logsumexp(scores, dim=-1)


def sdpa_fast(q, k, v):
    """Fused SDPA (torch's flash kernel on the CPU, its fp32 memory-efficient kernel on
    a GPU; no S x S materialisation) — used at full shapes (the CPU baseline, the
    full-size checks), where the chunked math path would be too slow."""
    return F.scaled_dot_product_attention(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)).squeeze(0)


def varlen_attention(q, k, v, cu_q, cu_k, attn=sdpa):
    """Block-diagonal varlen attention over packed [T, H, D] tensors.

    Segment m's queries [cu_q[m], cu_q[m+1]) attend only to keys
    [cu_k[m], cu_k[m+1]) — the semantics of the reference's varlen slot
    (sd35_batch.py:19-119,448-486) and of its per-segment fake
    (tests/python/test_domain_block_executor.py:869-883).
    """
    out = torch.empty(q.shape[:-1] + (v.shape[-1],), dtype=q.dtype, device=q.device)
    for m in range(len(cu_q) - 1):
        q0, q1, k0, k1 = cu_q[m], cu_q[m + 1], cu_k[m], cu_k[m + 1]
        if q1 == q0:
            continue
        o = attn(q[q0:q1].transpose(0, 1), k[k0:k1].transpose(0, 1), v[k0:k1].transpose(0, 1))
        out[q0:q1] = o.transpose(0, 1)
    return out

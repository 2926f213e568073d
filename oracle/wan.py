"""Oracle: Wan2.1 / Wan2.2 DiT transformer forward on CPU (fp32 or fp64).

Parameters are a dict keyed by diffusers WanTransformer3DModel state-dict
names ("blocks.3.attn1.to_q.weight", ...), every tensor already in the
compute dtype.  All activations stay in that dtype, so the `.type_as(h)` casts
of the reference are identities here (the reference's "CPU fp32" path).

Reference files followed:
  workers/ditserve/models/wan/block.py:276-297   (block arithmetic, _split_temb/_stage1/_stage2)
  workers/ditserve/models/wan/block.py:434-448   (prediction: norm_out, proj_out, unpatchify)
  workers/xfuser/model_executor/models/transformers/transformer_wan.py:50-69   (QKV projections)
  transformer_wan.py:79-156                        (processor: attention, to_out)
  transformer_wan.py:158-191                       (QK RMSNorm across heads + RoPE)
  transformer_wan.py:307-366                       (begin_packet: rope, patchify, condition embedder)
  transformer_wan.py:378-395                       (prediction)
  workers/ditserve/models/wan/runtime.py:153-163   (model_timestep)
"""
import math

import torch

from .common import gelu_tanh, layer_norm, linear, rms_norm, sdpa, silu, timestep_embedding, varlen_attention

ROPE_THETA = 10000.0


# ---------------------------------------------------------------------------
# RoPE (diffusers WanRotaryPosEmbed semantics, table built in float64 -> fp32)
# ---------------------------------------------------------------------------

def rope_axis_split(head_dim=128):
    """(t_dim, h_dim, w_dim) = (head_dim - 2*(2*(head_dim//6)), 2*(head_dim//6), 2*(head_dim//6))."""
    hw = 2 * (head_dim // 6)
    return head_dim - 2 * hw, hw, hw


def rope_table(head_dim=128, max_seq_len=1024, theta=ROPE_THETA):
    """freqs_cos / freqs_sin [max_seq_len, head_dim] fp32, concatenated t|h|w parts.

    Each part: freqs = 1 / theta^(arange(0, d, 2)/d), angles = outer(pos, freqs) in
    float64, cos/sin repeat-interleaved x2 and cast to float32.
    """
    pos = torch.arange(max_seq_len, dtype=torch.float64)
    cos_parts, sin_parts = [], []
    for d in rope_axis_split(head_dim):
        freqs = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64)[: d // 2] / d))
        ang = torch.outer(pos, freqs)
        cos_parts.append(ang.cos().repeat_interleave(2, dim=1).float())
        sin_parts.append(ang.sin().repeat_interleave(2, dim=1).float())
    return torch.cat(cos_parts, dim=1), torch.cat(sin_parts, dim=1)


def rope_freqs(grid, head_dim=128, max_seq_len=1024, theta=ROPE_THETA):
    """cos, sin [S, head_dim] fp32 for a (F', H', W') token grid, token order f-major then h then w."""
    f, h, w = grid
    cos_t, sin_t = rope_table(head_dim, max_seq_len, theta)
    td, hd, wd = rope_axis_split(head_dim)

    def expand(tab):
        a, b, c = tab.split([td, hd, wd], dim=1)
        a = a[:f].view(f, 1, 1, -1).expand(f, h, w, -1)
        b = b[:h].view(1, h, 1, -1).expand(f, h, w, -1)
        c = c[:w].view(1, 1, w, -1).expand(f, h, w, -1)
        return torch.cat([a, b, c], dim=-1).reshape(f * h * w, head_dim)

    return expand(cos_t), expand(sin_t)


def apply_rotary(x, cos, sin):
    """transformer_wan.py:170-188 — interleaved pairs: x [S, H, Dh], cos/sin [S, Dh].

    out[2i] = x[2i]*cos[2i] - x[2i+1]*sin[2i+1];  out[2i+1] = x[2i]*sin[2i+1] + x[2i+1]*cos[2i].
    """
    cos = cos.to(x.dtype)[:, None, :]
    sin = sin.to(x.dtype)[:, None, :]
    x1, x2 = x.unflatten(-1, (-1, 2)).unbind(-1)
    c = cos[..., 0::2]
    s = sin[..., 1::2]
    out = torch.empty_like(x)
    out[..., 0::2] = x1 * c - x2 * s
    out[..., 1::2] = x1 * s + x2 * c
    return out


def qk_norm_rope(q, k, wq, wk, cos, sin, heads, eps=1e-6):
    """transformer_wan.py:158-191 (also the `fused_qk_norm_rope` slot contract, :24-25,111-115).

    q, k [S, D] -> RMSNorm across all heads (affine) -> [S, H, Dh] -> RoPE (if cos is not None).
    """
    q = rms_norm(q, wq, eps).unflatten(-1, (heads, -1))
    k = rms_norm(k, wk, eps).unflatten(-1, (heads, -1))
    if cos is not None:
        q = apply_rotary(q, cos, sin)
        k = apply_rotary(k, cos, sin)
    return q, k


# ---------------------------------------------------------------------------
# block
# ---------------------------------------------------------------------------

def _attn_params(p, pre):
    g = lambda n: p[f"{pre}.{n}"]
    return g


def self_attention(p, pre, x, cos, sin, heads, eps=1e-6, attn=sdpa):
    """attn1: transformer_wan.py:50-69 (to_q/to_k/to_v), 158-191 (norm+rope), 138-155 (SDPA, to_out)."""
    g = _attn_params(p, pre)
    q = linear(x, g("to_q.weight"), g("to_q.bias"))
    k = linear(x, g("to_k.weight"), g("to_k.bias"))
    v = linear(x, g("to_v.weight"), g("to_v.bias"))
    q, k = qk_norm_rope(q, k, g("norm_q.weight"), g("norm_k.weight"), cos, sin, heads, eps)
    v = v.unflatten(-1, (heads, -1))
    o = attn(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)).transpose(0, 1).flatten(1)
    return linear(o, g("to_out.0.weight"), g("to_out.0.bias"))


def cross_attention(p, pre, x, enc, heads, eps=1e-6, attn=sdpa):
    """attn2: Q from image tokens, K/V from the text context; RMSNorm on q,k; no RoPE, no mask
    (zero-padded text rows attend) — transformer_wan.py:79-156 with use_ulysses=False (:244-246)."""
    g = _attn_params(p, pre)
    q = linear(x, g("to_q.weight"), g("to_q.bias"))
    k = linear(enc, g("to_k.weight"), g("to_k.bias"))
    v = linear(enc, g("to_v.weight"), g("to_v.bias"))
    q = rms_norm(q, g("norm_q.weight"), eps).unflatten(-1, (heads, -1))
    k = rms_norm(k, g("norm_k.weight"), eps).unflatten(-1, (heads, -1))
    v = v.unflatten(-1, (heads, -1))
    o = attn(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)).transpose(0, 1).flatten(1)
    return linear(o, g("to_out.0.weight"), g("to_out.0.bias"))


def split_modulation(p, i, projected):
    """block.py:276-280 (_split_temb): (scale_shift_table + projected).chunk(6).

    projected [6, D] (Wan2.1, one per request) -> 6 x [D]:
    shift_msa, scale_msa, gate_msa, c_shift_msa, c_scale_msa, c_gate_msa.
    """
    mod = p[f"blocks.{i}.scale_shift_table"].reshape(6, -1) + projected.reshape(6, -1)
    return mod.unbind(0)


def block_forward(p, i, hidden, encoder, projected, cos, sin, heads, eps=1e-6, attn=sdpa):
    """One Wan block on one request (block.py:276-297).

    hidden [S, D], encoder [L, D] (already text-embedded), projected [6, D],
    cos/sin [S, Dh].  Returns the new hidden [S, D].
    """
    pre = f"blocks.{i}"
    shift_msa, scale_msa, gate_msa, c_shift, c_scale, c_gate = split_modulation(p, i, projected)
    # _stage1 (block.py:282-285)
    n = layer_norm(hidden, eps) * (1.0 + scale_msa) + shift_msa
    a = self_attention(p, f"{pre}.attn1", n, cos, sin, heads, eps, attn)
    h = hidden + a * gate_msa
    # _stage2 (block.py:287-293)
    n = layer_norm(h, eps, p[f"{pre}.norm2.weight"], p[f"{pre}.norm2.bias"])
    h = h + cross_attention(p, f"{pre}.attn2", n, encoder, heads, eps, attn)
    n = layer_norm(h, eps) * (1.0 + c_scale) + c_shift
    f = linear(n, p[f"{pre}.ffn.net.0.proj.weight"], p[f"{pre}.ffn.net.0.proj.bias"])
    f = linear(gelu_tanh(f), p[f"{pre}.ffn.net.2.weight"], p[f"{pre}.ffn.net.2.bias"])
    return h + f * c_gate


def block_forward_packed(p, i, hidden, cu, encoders, projected, rotary, heads, eps=1e-6, attn=sdpa):
    """Packed block: segment m = hidden[cu[m]:cu[m+1]] runs block_forward with its own
    text context encoders[m], modulation projected[m] and rotary[m] = (cos, sin).
    The packed result is, by definition, the concatenation of per-request results."""
    out = torch.empty_like(hidden)
    for m in range(len(cu) - 1):
        s0, s1 = cu[m], cu[m + 1]
        cos, sin = rotary[m]
        out[s0:s1] = block_forward(p, i, hidden[s0:s1], encoders[m], projected[m], cos, sin, heads, eps, attn)
    return out


# ---------------------------------------------------------------------------
# packet prelude / epilogue
# ---------------------------------------------------------------------------

def model_timestep(latent_shape, t, expand):
    """runtime.py:153-163: Wan2.1 -> [B]; Wan2.2 TI2V -> per patch token [B, F*(H/2)*(W/2)]."""
    b, _, f, h, w = latent_shape
    if not expand:
        return torch.full((b,), float(t))
    return torch.full((b, f * (h // 2) * (w // 2)), float(t))


def condition_embedder(p, t, text, freq_dim=256):
    """diffusers WanTimeTextImageEmbedding as called at transformer_wan.py:331-333.

    t: [N] timesteps (one per request, or per token for Wan2.2); text [L, 4096].
    Returns temb [N, D], projected [N, 6, D], encoder [L, D].
    """
    pre = "condition_embedder"
    e = timestep_embedding(t, freq_dim).to(text.dtype)
    temb = linear(silu(linear(e, p[f"{pre}.time_embedder.linear_1.weight"], p[f"{pre}.time_embedder.linear_1.bias"])),
                  p[f"{pre}.time_embedder.linear_2.weight"], p[f"{pre}.time_embedder.linear_2.bias"])
    proj = linear(silu(temb), p[f"{pre}.time_proj.weight"], p[f"{pre}.time_proj.bias"])
    enc = linear(gelu_tanh(linear(text, p[f"{pre}.text_embedder.linear_1.weight"], p[f"{pre}.text_embedder.linear_1.bias"])),
                 p[f"{pre}.text_embedder.linear_2.weight"], p[f"{pre}.text_embedder.linear_2.bias"])
    return temb, proj.unflatten(-1, (6, -1)), enc


def patch_embed(p, latent, patch=(1, 2, 2)):
    """Conv3d(C, D, kernel=stride=patch) then flatten(2).transpose(1,2): latent [C, F, H, W] -> [S, D]."""
    c, f, h, w = latent.shape
    pt, ph, pw = patch
    x = latent.reshape(c, f // pt, pt, h // ph, ph, w // pw, pw)
    x = x.permute(1, 3, 5, 0, 2, 4, 6).reshape((f // pt) * (h // ph) * (w // pw), c * pt * ph * pw)
    wgt = p["patch_embedding.weight"].reshape(p["patch_embedding.weight"].shape[0], -1)
    return linear(x, wgt, p["patch_embedding.bias"])


def prediction(p, hidden, temb, grid, out_ch, patch=(1, 2, 2), eps=1e-6):
    """block.py:434-448 / transformer_wan.py:378-395: norm_out AdaLN with the model
    scale_shift_table [1,2,D] + temb, proj_out, unpatchify -> [C, F, H, W]."""
    shift, scale = (p["scale_shift_table"].reshape(2, -1) + temb.reshape(1, -1)).unbind(0)
    x = layer_norm(hidden, eps) * (1.0 + scale) + shift
    x = linear(x, p["proj_out.weight"], p["proj_out.bias"])
    f, h, w = grid
    pt, ph, pw = patch
    x = x.reshape(f, h, w, pt, ph, pw, out_ch).permute(6, 0, 3, 1, 4, 2, 5)
    return x.reshape(out_ch, f * pt, h * ph, w * pw)


def forward(p, cfg, latent, t, text, attn=sdpa, blocks=None):
    """Full transformer forward for one request / one CFG branch: latent [C, F, H, W],
    scalar timestep t, text [512, text_dim]. Returns the velocity prediction [C, F, H, W]."""
    pt, ph, pw = cfg["patch"]
    grid = (latent.shape[1] // pt, latent.shape[2] // ph, latent.shape[3] // pw)
    cos, sin = (x.to(latent.device) for x in rope_freqs(grid, cfg["head_dim"], cfg.get("rope_max_seq_len", 1024)))
    hidden = patch_embed(p, latent, cfg["patch"])
    temb, projected, enc = condition_embedder(p, torch.tensor([float(t)], device=latent.device), text,
                                              cfg["freq_dim"])
    n_blocks = cfg["layers"] if blocks is None else blocks
    for i in range(n_blocks):
        hidden = block_forward(p, i, hidden, enc, projected[0], cos, sin, cfg["heads"], cfg["eps"], attn)
    return prediction(p, hidden, temb[0], grid, cfg["out_ch"], cfg["patch"], cfg["eps"])


def cfg_combine(cond, uncond, guidance):
    """block.py:483 / runtime.py:689: uncond + g * (cond - uncond)."""
    return uncond + guidance * (cond - uncond)


def block_flops(s, d, heads, ffn, text_len):
    """Algorithmic FLOPs of one block forward over one request of s tokens."""
    proj = 2 * s * d * d * 4 + 2 * s * d * d * 2 + 2 * text_len * d * d * 2
    attn_self = 4 * s * s * d
    attn_cross = 4 * s * text_len * d
    ffn_f = 4 * s * d * ffn
    return proj + attn_self + attn_cross + ffn_f


def rope_pair_angle(pair, f, h, w, head_dim=128, theta=ROPE_THETA):
    """Closed form of the angle of rotation pair `pair` for token (f, h, w) (float64)."""
    td, hd, wd = rope_axis_split(head_dim)
    if pair < td // 2:
        return f * theta ** (-(2 * pair) / td)
    pair -= td // 2
    if pair < hd // 2:
        return h * theta ** (-(2 * pair) / hd)
    pair -= hd // 2
    return w * theta ** (-(2 * pair) / wd)


_ = math  # keep the import (used by callers via rope_pair_angle docs)

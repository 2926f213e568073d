"""Oracle: SD3.5-Medium MMDiT forward on CPU (fp32 or fp64), dense and packed.

Parameters are a dict keyed by diffusers SD3Transformer2DModel state-dict names,
already in the compute dtype.  Reference files followed:
  workers/ditserve/models/sd35_batch.py:336-376   (_packed_adaln_zero: 6 / 9 chunks)
  workers/ditserve/models/sd35_batch.py:379-393   (_packed_adaln_continuous: scale first)
  workers/ditserve/models/sd35_batch.py:396-495   (_packed_joint_attention, joint = image then text)
  workers/ditserve/models/sd35_batch.py:584-736   (forward_packed_sd35: block loop, dual attention,
                                                   FFNs, norm_out, proj_out, unpatchify)
  workers/xfuser/model_executor/layers/attention_processor.py:444-464 (joint attention at 1 GPU)
The diffusers modules themselves (PatchEmbed, CombinedTimestepTextProjEmbeddings,
JointTransformerBlock) are not in the reference tree: their restatement here is
"parity unpinned" beyond the in-tree call sites above.
"""
import math

import torch

from .common import gelu_tanh, layer_norm, linear, rms_norm, sdpa, silu, timestep_embedding


def sincos_1d(dim, pos):
    """[len(pos), dim]: [sin(pos * w_k), cos(pos * w_k)], w_k = 10000^(-k/(dim/2)) (float64)."""
    omega = torch.arange(dim // 2, dtype=torch.float64) / (dim / 2.0)
    omega = 1.0 / 10000 ** omega
    out = torch.outer(pos.reshape(-1).double(), omega)
    return torch.cat([torch.sin(out), torch.cos(out)], dim=1)


def pos_embed_table(dim, max_size=384, base_size=64, interpolation_scale=1.0):
    """[max_size^2, dim] fp32 2D sin-cos table: per (row h, column w) the first half
    encodes the column coordinate and the second half the row coordinate, with
    coordinates arange(n) / (n / base_size) / interpolation_scale."""
    coords = torch.arange(max_size, dtype=torch.float32) / (max_size / base_size) / interpolation_scale
    gw = coords.view(1, -1).expand(max_size, max_size)  # varies along columns
    gh = coords.view(-1, 1).expand(max_size, max_size)  # varies along rows
    return torch.cat([sincos_1d(dim // 2, gw), sincos_1d(dim // 2, gh)], dim=1).float()


def cropped_pos_embed(table, hp, wp):
    """Centre crop of a [max_size^2, dim] table for an hp x wp patch grid -> [hp*wp, dim]
    (max_size = pos_embed_max_size, read off the table: 384 for SD3.5-Medium, 192 for
    -Large)."""
    max_size = int(round(table.shape[0] ** 0.5))
    if max_size * max_size != table.shape[0] or hp > max_size or wp > max_size:
        raise ValueError(f"a {hp} x {wp} grid does not crop from a {table.shape[0]}-row table")
    top, left = (max_size - hp) // 2, (max_size - wp) // 2
    return table.view(max_size, max_size, -1)[top:top + hp, left:left + wp].reshape(hp * wp, -1)


def patch_embed(p, latent, table, patch=2):
    """Conv2d(C, D, k=s=patch) -> flatten -> + cropped pos embed: [C, H, W] -> [S, D]."""
    c, h, w = latent.shape
    x = latent.reshape(c, h // patch, patch, w // patch, patch).permute(1, 3, 0, 2, 4).reshape(-1, c * patch * patch)
    wgt = p["pos_embed.proj.weight"].reshape(p["pos_embed.proj.weight"].shape[0], -1)
    pos = cropped_pos_embed(table, h // patch, w // patch).to(device=x.device, dtype=x.dtype)
    return linear(x, wgt, p["pos_embed.proj.bias"]) + pos


def time_text_embed(p, t, pooled):
    """temb = TimestepEmbedding(sinusoid(t)) + PixArtAlphaTextProjection(pooled), [M, D]."""
    pre = "time_text_embed"
    e = timestep_embedding(t, 256).to(pooled.dtype)
    te = linear(silu(linear(e, p[f"{pre}.timestep_embedder.linear_1.weight"], p[f"{pre}.timestep_embedder.linear_1.bias"])),
                p[f"{pre}.timestep_embedder.linear_2.weight"], p[f"{pre}.timestep_embedder.linear_2.bias"])
    pe = linear(silu(linear(pooled, p[f"{pre}.text_embedder.linear_1.weight"], p[f"{pre}.text_embedder.linear_1.bias"])),
                p[f"{pre}.text_embedder.linear_2.weight"], p[f"{pre}.text_embedder.linear_2.bias"])
    return te + pe


def adaln_zero(p, pre, x, temb, eps=1e-6):
    """sd35_batch.py:336-376 for one segment: emb = Linear(SiLU(temb)) chunked 6 or 9."""
    emb = linear(silu(temb), p[f"{pre}.linear.weight"], p[f"{pre}.linear.bias"])
    d = x.shape[-1]
    chunks = emb.reshape(-1, d).unbind(0)
    nx = layer_norm(x, eps)
    out = {"normed": nx * (1.0 + chunks[1]) + chunks[0], "gate_msa": chunks[2], "shift_mlp": chunks[3],
           "scale_mlp": chunks[4], "gate_mlp": chunks[5]}
    if len(chunks) == 9:
        out["normed2"] = nx * (1.0 + chunks[7]) + chunks[6]
        out["gate_msa2"] = chunks[8]
    return out


def adaln_continuous(p, pre, x, temb, eps=1e-6):
    """sd35_batch.py:379-393: (scale, shift) = chunk(2) of Linear(SiLU(temb)); LN(x)(1+scale)+shift."""
    emb = linear(silu(temb), p[f"{pre}.linear.weight"], p[f"{pre}.linear.bias"])
    scale, shift = emb.reshape(2, -1).unbind(0)
    return layer_norm(x, eps) * (1.0 + scale) + shift


def _heads(x, heads):
    return x.unflatten(-1, (heads, -1))


def joint_attention(p, pre, x_img, x_txt, heads, context_pre_only, eps=1e-6, attn=sdpa):
    """One segment's joint attention (sd35_batch.py:410-495): image QKV + text add_q/k/v,
    per-head RMSNorm, joint sequence image-then-text, split, to_out / to_add_out."""
    g = lambda n: p[f"{pre}.{n}"]  # noqa: E731
    q = rms_norm(_heads(linear(x_img, g("to_q.weight"), g("to_q.bias")), heads), g("norm_q.weight"), eps)
    k = rms_norm(_heads(linear(x_img, g("to_k.weight"), g("to_k.bias")), heads), g("norm_k.weight"), eps)
    v = _heads(linear(x_img, g("to_v.weight"), g("to_v.bias")), heads)
    n = x_img.shape[0]
    if x_txt is not None:
        qt = rms_norm(_heads(linear(x_txt, g("add_q_proj.weight"), g("add_q_proj.bias")), heads), g("norm_added_q.weight"), eps)
        kt = rms_norm(_heads(linear(x_txt, g("add_k_proj.weight"), g("add_k_proj.bias")), heads), g("norm_added_k.weight"), eps)
        vt = _heads(linear(x_txt, g("add_v_proj.weight"), g("add_v_proj.bias")), heads)
        q, k, v = torch.cat([q, qt]), torch.cat([k, kt]), torch.cat([v, vt])
    o = attn(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1)).transpose(0, 1).flatten(1)
    img = linear(o[:n], g("to_out.0.weight"), g("to_out.0.bias"))
    txt = None
    if x_txt is not None and not context_pre_only:
        txt = linear(o[n:], g("to_add_out.weight"), g("to_add_out.bias"))
    return img, txt


def self_attention(p, pre, x, heads, eps=1e-6, attn=sdpa):
    """Dual (image-only) attention attn2 of the first blocks (sd35_batch.py:681-694)."""
    img, _ = joint_attention(p, pre, x, None, heads, True, eps, attn)
    return img


def ffn(p, pre, x):
    return linear(gelu_tanh(linear(x, p[f"{pre}.net.0.proj.weight"], p[f"{pre}.net.0.proj.bias"])),
                  p[f"{pre}.net.2.weight"], p[f"{pre}.net.2.bias"])


def joint_block(p, i, h, c, temb, cfg, attn=sdpa):
    """One JointTransformerBlock on one segment (sd35_batch.py:647-708 per segment).
    h [N, D] image tokens, c [L, D] text tokens, temb [D].  Returns (h, c or None)."""
    pre = f"transformer_blocks.{i}"
    heads, eps = cfg["heads"], cfg["eps"]
    pre_only = i == cfg["layers"] - 1
    dual = i in cfg["dual_layers"]
    a = adaln_zero(p, f"{pre}.norm1", h, temb, eps)
    if pre_only:
        nc = adaln_continuous(p, f"{pre}.norm1_context", c, temb, eps)
    else:
        ac = adaln_zero(p, f"{pre}.norm1_context", c, temb, eps)
        nc = ac["normed"]
    img, txt = joint_attention(p, f"{pre}.attn", a["normed"], nc, heads, pre_only, eps, attn)
    h = h + a["gate_msa"] * img
    if dual:
        h = h + a["gate_msa2"] * self_attention(p, f"{pre}.attn2", a["normed2"], heads, eps, attn)
    n2 = layer_norm(h, eps) * (1.0 + a["scale_mlp"]) + a["shift_mlp"]
    h = h + a["gate_mlp"] * ffn(p, f"{pre}.ff", n2)
    if pre_only:
        return h, None
    c = c + ac["gate_msa"] * txt
    n2c = layer_norm(c, eps) * (1.0 + ac["scale_mlp"]) + ac["shift_mlp"]
    c = c + ac["gate_mlp"] * ffn(p, f"{pre}.ff_context", n2c)
    return h, c


def forward(p, cfg, latent, t, text, pooled, attn=sdpa, table=None):
    """One request: latent [C, H, W], scalar t, text [L, 4096], pooled [2048] -> [C, H, W]."""
    table = pos_embed_table(cfg["dim"], cfg["pos_max"], cfg["base_size"]) if table is None else table
    h = patch_embed(p, latent, table, cfg["patch"])
    c = linear(text, p["context_embedder.weight"], p["context_embedder.bias"])
    temb = time_text_embed(p, torch.tensor([float(t)], device=latent.device), pooled.reshape(1, -1))[0]
    for i in range(cfg["layers"]):
        h, c = joint_block(p, i, h, c, temb, cfg, attn)
    x = adaln_continuous(p, "norm_out", h, temb, cfg["eps"])
    x = linear(x, p["proj_out.weight"], p["proj_out.bias"])
    ch, hh, ww = latent.shape
    ps = cfg["patch"]
    x = x.reshape(hh // ps, ww // ps, ps, ps, cfg["out_ch"]).permute(4, 0, 2, 1, 3)
    return x.reshape(cfg["out_ch"], hh, ww)


def forward_packed(p, cfg, latents, ts, texts, pooleds, attn=sdpa):
    """forward_packed_sd35 semantics (sd35_batch.py:584-736): the packed result is, by
    definition, each request's own forward."""
    table = pos_embed_table(cfg["dim"], cfg["pos_max"], cfg["base_size"])
    return [forward(p, cfg, lat, t, tx, po, attn, table) for lat, t, tx, po in zip(latents, ts, texts, pooleds)]


_ = math

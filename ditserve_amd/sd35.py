"""SD3.5-Medium MMDiT on the ditk HIP kernels, packed over variable resolutions.

Mirrors the reference's packed forward (workers/ditserve/models/sd35_batch.py:584-736):

  forward_packed_sd35(torch_mod, transformer, latents_list, timesteps_list,
                      encoder_hidden_states_list, pooled_projections_list) -> (outputs, meta)

Image tokens of all requests are packed into one [sum N_m, D] buffer and text
tokens into one [sum L_m, D] buffer; every projection, norm and FFN runs once
over the packed rows, modulation is gathered per token by segment, and joint
attention runs as one varlen flash launch over the joint layout (each segment's
image tokens followed by its text tokens, cu_joint[m] = cu_img[m] + cu_txt[m],
sd35_batch.py:230-317).  Each request's output is bitwise equal to its solo run.

Block (sd35_batch.py:647-708), per JointTransformerBlock:
  AdaLN-Zero (6 chunks, 9 with dual attention) on image and text, or
  AdaLN-Continuous (scale, shift) on text for the last (context_pre_only) block;
  joint attention with per-head QK RMSNorm; dual image-only attention (first
  blocks); gated residuals; GELU-tanh FFNs on image and text.
"""
import dataclasses
import math

import torch

from . import ops
from .ops import Segments
from .packing import joint_layout
from .profiling import NULL as _NULL_PROFILER

_BF16 = torch.bfloat16


@dataclasses.dataclass(frozen=True)
class SD35Config:
    dim: int = 1536
    heads: int = 24
    head_dim: int = 64
    layers: int = 24
    dual_layers: tuple = tuple(range(13))
    in_ch: int = 16
    out_ch: int = 16
    patch: int = 2
    text_dim: int = 4096
    pooled_dim: int = 2048
    ffn: int = 6144
    freq_dim: int = 256
    eps: float = 1e-6
    pos_max: int = 384
    base_size: int = 64

    @classmethod
    def from_diffusers(cls, config):
        """From a diffusers SD3Transformer2DModel config (a mapping or an object with
        attributes)."""
        get = config.get if isinstance(config, dict) else (lambda k, d=None: getattr(config, k, d))
        if get("qk_norm") != "rms_norm":
            raise ValueError("SD3.5 blocks here need qk_norm='rms_norm'")
        heads, hd = int(get("num_attention_heads")), int(get("attention_head_dim"))
        dim = heads * hd
        if int(get("caption_projection_dim")) != dim:
            raise ValueError("caption_projection_dim must equal the hidden size")
        patch = int(get("patch_size"))
        return cls(dim=dim, heads=heads, head_dim=hd, layers=int(get("num_layers")),
                   dual_layers=tuple(get("dual_attention_layers") or ()), in_ch=int(get("in_channels")),
                   out_ch=int(get("out_channels") or get("in_channels")), patch=patch,
                   text_dim=int(get("joint_attention_dim")), pooled_dim=int(get("pooled_projection_dim")),
                   ffn=4 * dim, pos_max=int(get("pos_embed_max_size")),
                   base_size=int(get("sample_size")) // patch)

    def oracle_dict(self):
        return dict(dim=self.dim, heads=self.heads, layers=self.layers, dual_layers=self.dual_layers,
                    eps=self.eps, patch=self.patch, out_ch=self.out_ch, pos_max=self.pos_max,
                    base_size=self.base_size)


SD35_MEDIUM = SD35Config()


def state_dict_shapes(cfg):
    """diffusers SD3Transformer2DModel parameter names and shapes."""
    D, F, P = cfg.dim, cfg.ffn, cfg.patch
    s = {
        "pos_embed.proj.weight": (D, cfg.in_ch, P, P), "pos_embed.proj.bias": (D,),
        "time_text_embed.timestep_embedder.linear_1.weight": (D, cfg.freq_dim),
        "time_text_embed.timestep_embedder.linear_1.bias": (D,),
        "time_text_embed.timestep_embedder.linear_2.weight": (D, D),
        "time_text_embed.timestep_embedder.linear_2.bias": (D,),
        "time_text_embed.text_embedder.linear_1.weight": (D, cfg.pooled_dim),
        "time_text_embed.text_embedder.linear_1.bias": (D,),
        "time_text_embed.text_embedder.linear_2.weight": (D, D),
        "time_text_embed.text_embedder.linear_2.bias": (D,),
        "context_embedder.weight": (D, cfg.text_dim), "context_embedder.bias": (D,),
        "norm_out.linear.weight": (2 * D, D), "norm_out.linear.bias": (2 * D,),
        "proj_out.weight": (P * P * cfg.out_ch, D), "proj_out.bias": (P * P * cfg.out_ch,),
    }
    for i in range(cfg.layers):
        b = f"transformer_blocks.{i}"
        last, dual = i == cfg.layers - 1, i in cfg.dual_layers
        s[f"{b}.norm1.linear.weight"] = ((9 if dual else 6) * D, D)
        s[f"{b}.norm1.linear.bias"] = ((9 if dual else 6) * D,)
        s[f"{b}.norm1_context.linear.weight"] = ((2 if last else 6) * D, D)
        s[f"{b}.norm1_context.linear.bias"] = ((2 if last else 6) * D,)
        names = ["to_q", "to_k", "to_v", "to_out.0", "add_q_proj", "add_k_proj", "add_v_proj"]
        if not last:
            names.append("to_add_out")
        for n in names:
            s[f"{b}.attn.{n}.weight"] = (D, D)
            s[f"{b}.attn.{n}.bias"] = (D,)
        for n in ("norm_q", "norm_k", "norm_added_q", "norm_added_k"):
            s[f"{b}.attn.{n}.weight"] = (cfg.head_dim,)
        if dual:
            for n in ("to_q", "to_k", "to_v", "to_out.0"):
                s[f"{b}.attn2.{n}.weight"] = (D, D)
                s[f"{b}.attn2.{n}.bias"] = (D,)
            for n in ("norm_q", "norm_k"):
                s[f"{b}.attn2.{n}.weight"] = (cfg.head_dim,)
        for ff in (["ff"] if last else ["ff", "ff_context"]):
            s[f"{b}.{ff}.net.0.proj.weight"] = (F, D)
            s[f"{b}.{ff}.net.0.proj.bias"] = (F,)
            s[f"{b}.{ff}.net.2.weight"] = (D, F)
            s[f"{b}.{ff}.net.2.bias"] = (D,)
    return s


def random_state_dict(cfg, seed=0, device="cpu", std=0.02):
    """Synthetic random init rounded to bf16 values (fp32 tensors): weights and biases
    N(0, std^2), RMSNorm weights N(1, std^2); deterministic per (seed, device)."""
    gen = torch.Generator(device=device).manual_seed(seed)
    sd = {}
    for name, shape in state_dict_shapes(cfg).items():
        t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std
        if ".norm_" in name:
            t = t + 1.0
        sd[name] = t.to(_BF16).float()
    return sd


def pos_embed_crop(cfg, hp, wp, device):
    """Cropped 2D sin-cos position table [hp*wp, D] (fp32): centre crop of the
    pos_max x pos_max grid with coordinates arange(n) * base_size / pos_max; the
    first half of each vector encodes the column, the second half the row."""
    top, left = (cfg.pos_max - hp) // 2, (cfg.pos_max - wp) // 2
    # fp32 coordinates i / (pos_max / base_size), as the table's grid is built
    coords = torch.arange(cfg.pos_max, dtype=torch.float32) / (cfg.pos_max / cfg.base_size)
    rows = coords[top:top + hp].double()
    cols = coords[left:left + wp].double()
    half = cfg.dim // 2
    omega = 1.0 / 10000 ** (torch.arange(half // 2, dtype=torch.float64) / (half / 2.0))

    def enc(pos):
        out = torch.outer(pos, omega)
        return torch.cat([torch.sin(out), torch.cos(out)], dim=1)

    ew = enc(cols).unsqueeze(0).expand(hp, wp, half)
    eh = enc(rows).unsqueeze(1).expand(hp, wp, half)
    return torch.cat([ew, eh], dim=-1).reshape(hp * wp, cfg.dim).float().to(device)


class SD35Transformer:
    """Device-resident SD3.5 MMDiT."""

    def __init__(self, cfg, state_dict, device="cuda"):
        self.cfg = cfg
        self.device = torch.device(device)
        dev, D, H = self.device, cfg.dim, cfg.heads

        def w(n):
            t = state_dict[n]
            return t.to(device=dev, dtype=_BF16).reshape(t.shape[0], -1).contiguous()

        def f(n):
            return state_dict[n].to(device=dev, dtype=torch.float32).contiguous()

        def per_head(n):  # per-head RMSNorm weight repeated over heads -> [D]
            return state_dict[n].to(device=dev, dtype=torch.float32).repeat(H).contiguous()

        self.pe_w, self.pe_b = w("pos_embed.proj.weight"), f("pos_embed.proj.bias")
        t = "time_text_embed"
        self.te1 = (w(f"{t}.timestep_embedder.linear_1.weight"), f(f"{t}.timestep_embedder.linear_1.bias"))
        self.te2 = (w(f"{t}.timestep_embedder.linear_2.weight"), f(f"{t}.timestep_embedder.linear_2.bias"))
        self.pp1 = (w(f"{t}.text_embedder.linear_1.weight"), f(f"{t}.text_embedder.linear_1.bias"))
        self.pp2 = (w(f"{t}.text_embedder.linear_2.weight"), f(f"{t}.text_embedder.linear_2.bias"))
        self.ctx = (w("context_embedder.weight"), f("context_embedder.bias"))
        self.norm_out = (w("norm_out.linear.weight"), f("norm_out.linear.bias"))
        self.proj_out = (w("proj_out.weight"), f("proj_out.bias"))
        if cfg.head_dim != 64:
            raise ValueError("the SD3.5 joint attention kernels take head_dim 64 (SD3.5 uses 64)")
        self._q_mult = ops.LOG2E / math.sqrt(cfg.head_dim)
        self.blocks = []
        for i in range(cfg.layers):
            b = f"transformer_blocks.{i}"
            a = f"{b}.attn"
            last, dual = i == cfg.layers - 1, i in cfg.dual_layers
            blk = {
                "last": last, "dual": dual,
                "n1": (w(f"{b}.norm1.linear.weight"), f(f"{b}.norm1.linear.bias")),
                "n1c": (w(f"{b}.norm1_context.linear.weight"), f(f"{b}.norm1_context.linear.bias")),
                "qkv": (torch.cat([w(f"{a}.to_q.weight"), w(f"{a}.to_k.weight"), w(f"{a}.to_v.weight")]),
                        torch.cat([f(f"{a}.to_q.bias"), f(f"{a}.to_k.bias"), f(f"{a}.to_v.bias")])),
                "qkv_t": (torch.cat([w(f"{a}.add_q_proj.weight"), w(f"{a}.add_k_proj.weight"),
                                     w(f"{a}.add_v_proj.weight")]),
                          torch.cat([f(f"{a}.add_q_proj.bias"), f(f"{a}.add_k_proj.bias"), f(f"{a}.add_v_proj.bias")])),
                "nq": per_head(f"{a}.norm_q.weight"), "nk": per_head(f"{a}.norm_k.weight"),
                "nqt": per_head(f"{a}.norm_added_q.weight"), "nkt": per_head(f"{a}.norm_added_k.weight"),
                "out": (w(f"{a}.to_out.0.weight"), f(f"{a}.to_out.0.bias")),
                "ff1": (w(f"{b}.ff.net.0.proj.weight"), f(f"{b}.ff.net.0.proj.bias")),
                "ff2": (w(f"{b}.ff.net.2.weight"), f(f"{b}.ff.net.2.bias")),
            }
            if not last:
                blk["out_t"] = (w(f"{a}.to_add_out.weight"), f(f"{a}.to_add_out.bias"))
                blk["ffc1"] = (w(f"{b}.ff_context.net.0.proj.weight"), f(f"{b}.ff_context.net.0.proj.bias"))
                blk["ffc2"] = (w(f"{b}.ff_context.net.2.weight"), f(f"{b}.ff_context.net.2.bias"))
            if dual:
                a2 = f"{b}.attn2"
                blk["qkv2"] = (torch.cat([w(f"{a2}.to_q.weight"), w(f"{a2}.to_k.weight"), w(f"{a2}.to_v.weight")]),
                               torch.cat([f(f"{a2}.to_q.bias"), f(f"{a2}.to_k.bias"), f(f"{a2}.to_v.bias")]))
                blk["nq2"], blk["nk2"] = per_head(f"{a2}.norm_q.weight"), per_head(f"{a2}.norm_k.weight")
                blk["out2"] = (w(f"{a2}.to_out.0.weight"), f(f"{a2}.to_out.0.bias"))
            # the q-side RMSNorm weights carry softmax_scale * log2(e), so the normed
            # q leaves the norm kernel pre-scaled (still one bf16 rounding) and
            # attention skips its per-score scaling
            for key in ("nq", "nqt", "nq2"):
                if key in blk:
                    blk[key + "_pre"] = blk[key] * self._q_mult
            self.blocks.append(blk)
        # Every AdaLN modulation projection (norm1, norm1_context of each block,
        # norm_out) reads the same conditioning rows silu(temb), so all of them
        # run as one GEMM per step over the weights stacked along N: one launch
        # streams the ~1.5 GB of modulation weights instead of 49 launches with
        # two rows each.  Per-layer entries become views into the stacked copy.
        mods = [(blk, key) for blk in self.blocks for key in ("n1", "n1c")]
        parts = [blk[key] for blk, key in mods] + [self.norm_out]
        self.mod_w = torch.cat([p[0] for p in parts])
        self.mod_b = torch.cat([p[1] for p in parts])
        off = 0
        for (blk, key), (pw, _) in zip(mods, parts):
            n = pw.shape[0]
            blk[key] = (self.mod_w[off:off + n], self.mod_b[off:off + n])
            blk[key + "_cols"] = (off, off + n)
            off += n
        n = self.norm_out[0].shape[0]
        self.norm_out = (self.mod_w[off:off + n], self.mod_b[off:off + n])
        self.norm_out_cols = (off, off + n)
        del parts
        self._pos_cache = {}
        self.profiler = _NULL_PROFILER

    @classmethod
    def random(cls, cfg, seed=0, device="cuda"):
        return cls(cfg, random_state_dict(cfg, seed, device), device)

    def _pos(self, hp, wp):
        key = (hp, wp)
        if key not in self._pos_cache:
            self._pos_cache[key] = pos_embed_crop(self.cfg, hp, wp, self.device).to(_BF16)
        return self._pos_cache[key]

    # ------------------------------------------------------------------ pieces
    def _attention(self, qkv, seg, wq, wk):
        """Per-head QK RMSNorm (in place on the qkv buffer) + varlen flash over seg
        (wq carries the softmax pre-scale)."""
        D, H, Dh = self.cfg.dim, self.cfg.heads, self.cfg.head_dim
        q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
        ops.qk_norm_rope_(q, k, wq, wk, Dh, self.cfg.eps, per_head=True)
        with self.profiler.region("attn_dual_core"):
            return ops.flash_attn_varlen(q, k, v, seg, seg, H, Dh, q_prescaled=True)

    def _block(self, i, h, c, mod, seg_img, seg_txt, seg_joint):
        cfg, blk, prof = self.cfg, self.blocks[i], self.profiler
        D, eps = cfg.dim, cfg.eps
        with prof.region("adaln"):
            # image AdaLN-Zero (and the dual branch's), text AdaLN-Zero or, in the last
            # block, AdaLN-Continuous (scale, shift): one launch
            emb = mod[:, slice(*blk["n1_cols"])]  # [M, 6D or 9D]
            embc = mod[:, slice(*blk["n1c_cols"])]  # [M, 2D] (last) or [M, 6D]
            jobs = [dict(x=h, shift=emb[:, 0:D], scale=emb[:, D:2 * D], segments=seg_img, eps=eps)]
            if blk["last"]:
                jobs.append(dict(x=c, shift=embc[:, D:2 * D], scale=embc[:, 0:D], segments=seg_txt, eps=eps))
            else:
                jobs.append(dict(x=c, shift=embc[:, 0:D], scale=embc[:, D:2 * D], segments=seg_txt, eps=eps))
            if blk["dual"]:
                jobs.append(dict(x=h, shift=emb[:, 6 * D:7 * D], scale=emb[:, 7 * D:8 * D], segments=seg_img, eps=eps))
            normed = ops.adaln_multi(jobs)
            nh, nc = normed[0], normed[1]
            nh2 = normed[2] if blk["dual"] else None
        with prof.region("gemm_qkv"):
            with prof.region("gemm_qkv_img"):
                qkv_i = ops.linear(nh, *blk["qkv"])
            with prof.region("gemm_qkv_txt"):
                qkv_t = ops.linear(nc, *blk["qkv_t"])
        with prof.region("joint_prep"):
            D3 = 3 * D
            with prof.region("qk_norm"):  # image and text per-head QK RMSNorm, in place, one launch
                ops.qk_norm_multi([
                    dict(q=qkv_i[:, :D], k=qkv_i[:, D:2 * D], wq=blk["nq_pre"], wk=blk["nk"], head_dim=cfg.head_dim,
                         eps=eps, per_head=True),
                    dict(q=qkv_t[:, :D], k=qkv_t[:, D:2 * D], wq=blk["nqt_pre"], wk=blk["nkt"],
                         head_dim=cfg.head_dim, eps=eps, per_head=True)])
            # image and text rows are read in place: no gather / scatter copies
            with prof.region("transpose_v_joint"):
                vt = ops.transpose_v_joint(qkv_i[:, 2 * D:D3], qkv_t[:, 2 * D:D3], cfg.heads, cfg.head_dim,
                                           seg_img, seg_txt, seg_joint)
        with prof.region("attn_joint"):
            a_img, a_txt = ops.joint_attention_q_prescaled(
                qkv_i[:, :D], qkv_t[:, :D], qkv_i[:, D:2 * D], qkv_t[:, D:2 * D], vt, seg_img, seg_txt,
                seg_joint, cfg.heads, cfg.head_dim)
        with prof.region("gemm_out"):
            img = dict(x=a_img, w=blk["out"][0], b=blk["out"][1], residual=h, gate=emb[:, 2 * D:3 * D],
                       segments=seg_img)
            if blk["last"]:
                h = ops.linear(epilogue="gate_res", **img)
            else:  # image and text output projections, one launch where that pays
                with prof.region("gemm_out_pair"):
                    h, c = ops.linear_pair(img, dict(x=a_txt, w=blk["out_t"][0], b=blk["out_t"][1], residual=c,
                                                     gate=embc[:, 2 * D:3 * D], segments=seg_txt), "gate_res")
        if blk["dual"]:
            with prof.region("attn_dual"):
                qkv2 = ops.linear(nh2, *blk["qkv2"])
                a2 = self._attention(qkv2, seg_img, blk["nq2_pre"], blk["nk2"])
                ops.linear(a2, *blk["out2"], "gate_res", residual=h, gate=emb[:, 8 * D:9 * D], segments=seg_img, out=h)
        with prof.region("ffn"):
            jobs = [dict(x=h, shift=emb[:, 3 * D:4 * D], scale=emb[:, 4 * D:5 * D], segments=seg_img, eps=eps)]
            if not blk["last"]:
                jobs.append(dict(x=c, shift=embc[:, 3 * D:4 * D], scale=embc[:, 4 * D:5 * D], segments=seg_txt,
                                 eps=eps))
            normed = ops.adaln_multi(jobs)
            n2 = normed[0]
            with prof.region("gemm_ffn_up_img"):
                fx = ops.linear(n2, *blk["ff1"], "gelu")
            img = dict(x=fx, w=blk["ff2"][0], b=blk["ff2"][1], residual=h, gate=emb[:, 5 * D:6 * D],
                       segments=seg_img, out=h)
            if blk["last"]:
                ops.linear(epilogue="gate_res", **img)
                return h, None
            fc = ops.linear(normed[1], *blk["ffc1"], "gelu")
            with prof.region("gemm_ffn_down_pair"):
                ops.linear_pair(img, dict(x=fc, w=blk["ffc2"][0], b=blk["ffc2"][1], residual=c,
                                          gate=embc[:, 5 * D:6 * D], segments=seg_txt, out=c), "gate_res")
        return h, c

    # ------------------------------------------------------------------ forward
    def forward_packed(self, latents, timesteps, texts, pooleds):
        """latents: list of [C, H, W] (or [1, C, H, W]); timesteps: list of scalars;
        texts: list of [L, text_dim]; pooleds: list of [pooled_dim].
        Returns (list of fp32 [C, H, W], meta)."""
        cfg, dev, D = self.cfg, self.device, self.cfg.dim
        n = len(latents)
        if n == 0:
            raise ValueError("forward_packed requires at least one item")
        if not (len(timesteps) == len(texts) == len(pooleds) == n):
            raise ValueError("all input lists must have matching lengths")
        P = cfg.patch
        lats = [l.reshape(l.shape[-3:]) for l in latents]
        hw = []
        for l in lats:
            if l.shape[0] != cfg.in_ch or l.shape[1] % P or l.shape[2] % P:
                raise ValueError(f"latent {tuple(l.shape)} must be [{cfg.in_ch}, H, W] with H, W divisible by {P}")
            if max(l.shape[1], l.shape[2]) // P > cfg.pos_max:
                raise ValueError(f"latent {tuple(l.shape)} has more than pos_embed_max_size = {cfg.pos_max} patches "
                                 "along a side")
            hw.append((l.shape[1] // P, l.shape[2] // P))
        img_counts = [a * b for a, b in hw]
        for t in texts:
            if t.dim() < 2 or t.shape[-1] != cfg.text_dim:
                raise ValueError(f"text contexts must be [L, {cfg.text_dim}], got {tuple(t.shape)}")
        txts = [t.reshape(-1, cfg.text_dim) for t in texts]
        txt_counts = [t.shape[0] for t in txts]
        lay = joint_layout(img_counts, txt_counts)
        seg_img, seg_txt = Segments(lay["cu_img"], dev), Segments(lay["cu_txt"], dev)
        seg_joint = Segments(lay["cu_joint"], dev)
        # prelude: patch embed (+ cropped 2D sin-cos positions), context embedder, temb
        h = torch.empty((seg_img.total, D), dtype=_BF16, device=dev)
        for m, (l, (hp, wp)) in enumerate(zip(lats, hw)):
            patches = ops.patchify(l.reshape(cfg.in_ch, 1, *l.shape[1:]).to(_BF16), (1, P, P))
            rows = h[seg_img.cu[m]:seg_img.cu[m + 1]]
            ops.linear(patches, self.pe_w, self.pe_b, "res", residual=self._pos(hp, wp), out=rows)
        c = ops.linear(torch.cat([t.to(device=dev, dtype=_BF16) for t in txts]), *self.ctx)
        t = ops.to_device([float(x) for x in timesteps], torch.float32, dev)
        te = ops.linear(ops.linear(ops.timestep_embedding(t, cfg.freq_dim), *self.te1, "silu"), *self.te2)
        pooled = torch.stack([p.reshape(-1) for p in pooleds]).to(device=dev, dtype=_BF16)
        temb = ops.linear(ops.linear(pooled, *self.pp1, "silu"), *self.pp2, "res", residual=te)
        st = ops.silu(temb)
        mod = ops.linear(st, self.mod_w, self.mod_b, "f32")  # every block's modulation + norm_out
        for i in range(cfg.layers):
            h, c = self._block(i, h, c, mod, seg_img, seg_txt, seg_joint)
        # epilogue: AdaLN-Continuous norm_out (scale, shift), proj_out, per-request unpatchify
        embo = mod[:, slice(*self.norm_out_cols)]
        x = ops.adaln(h, embo[:, D:2 * D], embo[:, 0:D], seg_img, eps=cfg.eps)
        y = ops.linear(x, *self.proj_out)
        outs = []
        for m, (hp, wp) in enumerate(hw):
            u = ops.unpatchify(y[seg_img.cu[m]:seg_img.cu[m + 1]], (1, hp, wp), (1, P, P), cfg.out_ch)
            outs.append(u.reshape(cfg.out_ch, hp * P, wp * P))
        meta = {
            "sequence_packed": True,
            "attention_backend": "ditk_flash_varlen",
            "attention_provider": "ditk",
            "packed_segments": n,
            "cu_seqlens_img": lay["cu_img"],
            "cu_seqlens_txt": lay["cu_txt"],
            "cu_seqlens_joint": lay["cu_joint"],
            "packed_image_tokens": lay["cu_img"][-1],
            "padded_image_tokens": n * max(img_counts),
            "padding_saved_tokens": n * max(img_counts) - lay["cu_img"][-1],
        }
        return outs, meta

    def forward(self, hidden_states, timestep, encoder_hidden_states, pooled_projections):
        """Dense batch (e.g. the homogeneous CFG batch of workers/ditserve/models/sd35.py:956-1017):
        hidden_states [B, C, H, W] -> [B, C, H, W] fp32."""
        b = hidden_states.shape[0]
        ts = timestep.reshape(-1).tolist() if torch.is_tensor(timestep) else list(timestep)
        if len(ts) == 1:
            ts = ts * b
        outs, _ = self.forward_packed([hidden_states[i] for i in range(b)], ts,
                                      [encoder_hidden_states[i] for i in range(b)],
                                      [pooled_projections[i] for i in range(b)])
        return torch.stack(outs)


def forward_packed_sd35(torch_mod, transformer, latents_list, timesteps_list, encoder_hidden_states_list,
                        pooled_projections_list):
    """Signature of the reference's packed forward (sd35_batch.py:584-591); ``torch_mod``
    is accepted for call compatibility and ``transformer`` is an SD35Transformer.
    Latents are [1, C, h, w] each; returns ([1, C, h, w] outputs, meta)."""
    for lat in latents_list:
        if lat.ndim != 4 or lat.shape[0] != 1:
            raise ValueError("each latent in latents_list must have shape [1, C, H_lat, W_lat]")
    for enc in encoder_hidden_states_list:
        if enc.ndim != 3 or enc.shape[0] != 1:
            raise ValueError("each encoder_hidden_states item must have shape [1, L, D_ctx]")
    outs, meta = transformer.forward_packed(latents_list, [float(t.reshape(-1)[0]) if torch.is_tensor(t) else float(t)
                                                           for t in timesteps_list],
                                            encoder_hidden_states_list, pooled_projections_list)
    return [o.unsqueeze(0) for o in outs], meta


def step_flops(cfg, img_counts, txt_counts):
    """Algorithmic FLOPs of the transformer blocks for one packed forward."""
    D, F = cfg.dim, cfg.ffn
    total = 0
    for i in range(cfg.layers):
        last, dual = i == cfg.layers - 1, i in cfg.dual_layers
        for n, l in zip(img_counts, txt_counts):
            total += 2 * n * D * 3 * D + 2 * l * D * 3 * D          # QKV image + text
            total += 4 * (n + l) ** 2 * D                           # joint attention
            total += 2 * n * D * D + (0 if last else 2 * l * D * D)  # to_out / to_add_out
            total += 4 * n * D * F + (0 if last else 4 * l * D * F)  # FFNs
            if dual:
                total += 2 * n * D * 3 * D + 4 * n * n * D + 2 * n * D * D
    return total


def step_members_once(model, states, *, force_packing=False):
    """One denoising step of every state (mixed timesteps, resolutions, prompt
    lengths and CFG), as workers/ditserve/models/sd35.py:895-1020 does it: a CFG
    state contributes its unconditional then its conditional segment, and each
    state's scheduler steps on the CFG-combined output.  Every batch runs as one
    packed forward on the ditk kernels (a homogeneous batch is the packed batch of
    equal segments); the returned meta says which form the reference would take.

    A state is a dict with ``latents`` [1, C, h, w] fp32, ``timesteps``, ``step``,
    ``spec`` (``height``, ``width``, ``guidance_scale``), ``embeds``
    (``prompt_embeds`` [1, L, text_dim], ``pooled_prompt_embeds`` [1, pooled_dim]
    and their ``negative_`` forms for CFG) and ``scheduler`` (a
    FlowMatchEulerScheduler)."""
    resolutions = [(int(st["spec"]["height"]), int(st["spec"]["width"])) for st in states]
    cfg_flags = [float(st["spec"]["guidance_scale"]) > 1.0 for st in states]
    txt_lens = [int(st["embeds"]["prompt_embeds"].shape[1]) for st in states]
    use_packing = bool(force_packing or len(set(resolutions)) > 1 or len(set(cfg_flags)) > 1
                       or len(set(txt_lens)) > 1)
    lats, ts, encs, pooled, seg_map = [], [], [], [], []
    for idx, st in enumerate(states):
        t = st["timesteps"][int(st["step"])]
        emb = st["embeds"]
        s_uncond = None
        if cfg_flags[idx]:
            s_uncond = len(lats)
            lats.append(st["latents"])
            ts.append(t)
            encs.append(emb["negative_prompt_embeds"])
            pooled.append(emb["negative_pooled_prompt_embeds"])
        seg_map.append((idx, s_uncond, len(lats)))
        lats.append(st["latents"])
        ts.append(t)
        encs.append(emb["prompt_embeds"])
        pooled.append(emb["pooled_prompt_embeds"])
    outs, meta = forward_packed_sd35(torch, model, lats, ts, encs, pooled)
    for idx, s_uncond, s_cond in seg_map:
        st = states[idx]
        t = st["timesteps"][int(st["step"])]
        guidance = float(st["spec"]["guidance_scale"])
        uncond = outs[s_uncond] if s_uncond is not None else None
        st["latents"] = st["scheduler"].step(outs[s_cond], t, st["latents"], return_dict=False, uncond=uncond,
                                             guidance=guidance if uncond is not None else 1.0)[0]
        st["step"] = int(st["step"]) + 1
    if use_packing:
        return meta
    return {"sequence_packed": False, "vector_timesteps": [float(st["timesteps"][int(st["step"]) - 1])
                                                           for st in states], "batch_size": len(states)}


def advance_batch(model, states, state_ids, steps=1, *, sequence_packing=False, vae_scale_factor=8):
    """Advance 1..8 states by ``steps`` denoising steps in shared packed forwards and
    report the result in the shape of the reference's batched advance
    (workers/ditserve/models/sd35.py:1025-1164): per-state progress, the wall time
    (``model_ms``), the batch's packing summary, the last step's meta."""
    import time

    from .executor import memory, progress
    from .packing import packing_stats

    if not isinstance(state_ids, list) or not 1 <= len(state_ids) <= 8 or len(set(state_ids)) != len(state_ids):
        raise ValueError("advance_batch requires 1 to 8 distinct state_ids")
    if len(states) != len(state_ids):
        raise ValueError("one state per state id")
    if type(steps) is not int or steps < 1:
        raise ValueError("steps must be a positive integer")
    for sid, st in zip(state_ids, states):
        if int(st.get("step", 0)) >= int(st.get("steps", st["spec"]["steps"])):
            raise ValueError(f"state {sid} has already completed")
    torch.cuda.synchronize()
    started = time.perf_counter()
    step_meta = {}
    for st in states:
        st["steps"] = int(st.get("steps", st["spec"]["steps"]))
        st["step"] = int(st.get("step", 0))
    for _ in range(steps):
        active = [st for st in states if int(st["step"]) < int(st["steps"])]
        if not active:
            break
        step_meta = step_members_once(model, active, force_packing=sequence_packing)
    torch.cuda.synchronize()
    elapsed_ms = (time.perf_counter() - started) * 1000.0
    pack = packing_stats([int(st["spec"]["height"]) for st in states], [int(st["spec"]["width"]) for st in states],
                         vae_scale_factor=vae_scale_factor, patch_size=model.cfg.patch)
    results = []
    for sid, st in zip(state_ids, states):
        st["paused"] = int(st["step"]) < int(st["steps"])
        results.append(dict(state_id=sid, progress=progress(int(st["step"]), int(st["steps"])), paused=st["paused"]))
    return dict(results=results, batch_size=len(state_ids), quantum="continuous_batch", model_ms=round(elapsed_ms, 3),
                attention="ditk", bubble_free=False, sequence_packing=bool(step_meta.get("sequence_packed", False)),
                packing=pack, step_meta=step_meta, memory_after=memory())

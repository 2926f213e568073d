"""Wan2.1 / Wan2.2 DiT transformer on the ditk HIP kernels, behind the
reference's packet API.

Mirrors xFuserWanTransformer3DWrapper's packet surface
(workers/xfuser/model_executor/models/transformers/transformer_wan.py:307-418):

  begin_packet(hidden_states, timestep, encoder_hidden_states) -> packet dict
  forward_block(packet, index) -> new hidden (also stored in packet["hidden"])
  prediction(packet) -> velocity [B, C, F, H, W]
  forward(...) = begin_packet + every forward_block + prediction

and adds step-level packing: ``begin_packed_packet`` takes a list of requests
(latent, timestep, text context) — different grids, timesteps and texts — and
runs them as one varlen token batch.  Each request's slice of the packed
result is bitwise equal to running that request alone.

Block arithmetic follows workers/ditserve/models/wan/block.py:276-297:
  n  = LN(h) * (1 + scale_msa) + shift_msa                  (fused AdaLN kernel)
  q,k,v = n W_qkv^T + b                                      (one MFMA GEMM, N = 3D)
  q,k = RoPE(RMSNorm_D(q)), RoPE(RMSNorm_D(k))               (fused QK-norm+RoPE kernel)
  h  = h + O(attn(q,k,v)) * gate_msa                         (flash kernel; GEMM gate epilogue)
  n  = LN_affine(h); h = h + O(cross_attn(n, text))          (flash kernel; GEMM residual epilogue)
  n  = LN(h) * (1 + c_scale) + c_shift
  h  = h + W2 GELU_tanh(W1 n) * c_gate                       (GELU epilogue; gate epilogue)
"""
import dataclasses
import math
import weakref

import torch

from . import ops
from .ops import Segments
from .profiling import NULL as _NULL_PROFILER

_BF16 = torch.bfloat16


@dataclasses.dataclass(frozen=True)
class WanConfig:
    dim: int = 1536
    heads: int = 12
    head_dim: int = 128
    ffn: int = 8960
    layers: int = 30
    in_ch: int = 16
    out_ch: int = 16
    text_dim: int = 4096
    text_len: int = 512
    freq_dim: int = 256
    patch: tuple = (1, 2, 2)
    eps: float = 1e-6
    rope_max_seq_len: int = 1024
    rope_theta: float = 10000.0

    def as_dict(self):
        return dataclasses.asdict(self)

    @classmethod
    def from_diffusers(cls, config, text_len=512):
        """From a diffusers WanTransformer3DModel config (a mapping or an object with
        attributes): the keys its constructor takes.  ``text_len`` is the
        pipeline's padded prompt length, not part of that config."""
        get = config.get if isinstance(config, dict) else (lambda k, d=None: getattr(config, k, d))
        if get("added_kv_proj_dim") is not None or get("image_dim") is not None:
            raise ValueError("only text-to-video Wan transformers (no image conditioning) are supported")
        if get("qk_norm", "rms_norm_across_heads") != "rms_norm_across_heads" or not get("cross_attn_norm", True):
            raise ValueError("Wan blocks need qk_norm='rms_norm_across_heads' and cross_attn_norm=True")
        heads, hd = int(get("num_attention_heads")), int(get("attention_head_dim"))
        return cls(dim=heads * hd, heads=heads, head_dim=hd, ffn=int(get("ffn_dim")), layers=int(get("num_layers")),
                   in_ch=int(get("in_channels")), out_ch=int(get("out_channels")), text_dim=int(get("text_dim")),
                   text_len=text_len, freq_dim=int(get("freq_dim")), patch=tuple(get("patch_size")),
                   eps=float(get("eps")), rope_max_seq_len=int(get("rope_max_seq_len")))


WAN21_T2V_1_3B = WanConfig()
WAN22_TI2V_5B = WanConfig(dim=3072, heads=24, ffn=14336, in_ch=48, out_ch=48)
# the published Wan2.1-T2V-14B transformer config (workers/ditserve/evaluation/cost_profile.py:19-20)
WAN21_T2V_14B = WanConfig(dim=5120, heads=40, ffn=13824, layers=40)


# ---------------------------------------------------------------------------
# RoPE tables (WanRotaryPosEmbed semantics, float64 angles -> fp32)
# ---------------------------------------------------------------------------

def rope_axis_pairs(head_dim):
    """Rotation pairs owned by the frame, row and column axes: (t, h, w)."""
    hw = 2 * (head_dim // 6)
    t = head_dim - 2 * hw
    return t // 2, hw // 2, hw // 2


def rope_tables(head_dim, max_pos, theta, device):
    """cos/sin [max_pos, head_dim/2] fp32: entry [p, i] is the rotation of pair i
    at position p on the axis that owns pair i (angle = p * theta^(-2j/d_axis))."""
    tp, hp, wp = rope_axis_pairs(head_dim)
    pos = torch.arange(max_pos, dtype=torch.float64)
    cols = []
    for npairs in (tp, hp, wp):
        d = 2 * npairs
        freqs = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float64)[:npairs] / d))
        cols.append(torch.outer(pos, freqs))
    ang = torch.cat(cols, dim=1)
    return ang.cos().float().to(device), ang.sin().float().to(device)


# ---------------------------------------------------------------------------
# weights
# ---------------------------------------------------------------------------

def state_dict_shapes(cfg):
    """diffusers WanTransformer3DModel parameter names and shapes."""
    D, F, P = cfg.dim, cfg.ffn, cfg.patch
    shapes = {
        "patch_embedding.weight": (D, cfg.in_ch, *P),
        "patch_embedding.bias": (D,),
        "condition_embedder.time_embedder.linear_1.weight": (D, cfg.freq_dim),
        "condition_embedder.time_embedder.linear_1.bias": (D,),
        "condition_embedder.time_embedder.linear_2.weight": (D, D),
        "condition_embedder.time_embedder.linear_2.bias": (D,),
        "condition_embedder.time_proj.weight": (6 * D, D),
        "condition_embedder.time_proj.bias": (6 * D,),
        "condition_embedder.text_embedder.linear_1.weight": (D, cfg.text_dim),
        "condition_embedder.text_embedder.linear_1.bias": (D,),
        "condition_embedder.text_embedder.linear_2.weight": (D, D),
        "condition_embedder.text_embedder.linear_2.bias": (D,),
        "scale_shift_table": (1, 2, D),
        "proj_out.weight": (cfg.out_ch * P[0] * P[1] * P[2], D),
        "proj_out.bias": (cfg.out_ch * P[0] * P[1] * P[2],),
    }
    for i in range(cfg.layers):
        b = f"blocks.{i}"
        shapes[f"{b}.scale_shift_table"] = (1, 6, D)
        for a in ("attn1", "attn2"):
            for n in ("to_q", "to_k", "to_v", "to_out.0"):
                shapes[f"{b}.{a}.{n}.weight"] = (D, D)
                shapes[f"{b}.{a}.{n}.bias"] = (D,)
            shapes[f"{b}.{a}.norm_q.weight"] = (D,)
            shapes[f"{b}.{a}.norm_k.weight"] = (D,)
        shapes[f"{b}.norm2.weight"] = (D,)
        shapes[f"{b}.norm2.bias"] = (D,)
        shapes[f"{b}.ffn.net.0.proj.weight"] = (F, D)
        shapes[f"{b}.ffn.net.0.proj.bias"] = (F,)
        shapes[f"{b}.ffn.net.2.weight"] = (D, F)
        shapes[f"{b}.ffn.net.2.bias"] = (D,)
    return shapes


def random_state_dict(cfg, seed=0, device="cpu", std=0.02):
    """Synthetic random-init weights, rounded to bf16 values (returned fp32).

    Linear weights, biases and modulation tables ~ N(0, std^2); affine norm
    weights ~ N(1, std^2) so the norms keep unit scale.  Deterministic for a
    (seed, device) pair; tensors are drawn in state-dict order."""
    gen = torch.Generator(device=device).manual_seed(seed)
    sd = {}
    for name, shape in state_dict_shapes(cfg).items():
        t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std
        if name.endswith("norm_q.weight") or name.endswith("norm_k.weight") or name.endswith("norm2.weight"):
            t = t + 1.0
        sd[name] = t.to(_BF16).float()
    return sd


class WanTransformer:
    """Device-resident Wan transformer driven through the packet API."""

    def __init__(self, cfg, state_dict, device="cuda"):
        self.cfg = cfg
        self.device = torch.device(device)
        dev = self.device

        def w(name):  # bf16 GEMM weight, [N, K]
            return state_dict[name].to(device=dev, dtype=_BF16).reshape(state_dict[name].shape[0], -1).contiguous()

        def f(name):  # fp32 vector / table
            return state_dict[name].to(device=dev, dtype=torch.float32).contiguous()

        D = cfg.dim
        self.patch_w, self.patch_b = w("patch_embedding.weight"), f("patch_embedding.bias")
        ce = "condition_embedder"
        self.te1_w, self.te1_b = w(f"{ce}.time_embedder.linear_1.weight"), f(f"{ce}.time_embedder.linear_1.bias")
        self.te2_w, self.te2_b = w(f"{ce}.time_embedder.linear_2.weight"), f(f"{ce}.time_embedder.linear_2.bias")
        self.tp_w, self.tp_b = w(f"{ce}.time_proj.weight"), f(f"{ce}.time_proj.bias")
        self.tx1_w, self.tx1_b = w(f"{ce}.text_embedder.linear_1.weight"), f(f"{ce}.text_embedder.linear_1.bias")
        self.tx2_w, self.tx2_b = w(f"{ce}.text_embedder.linear_2.weight"), f(f"{ce}.text_embedder.linear_2.bias")
        self.sst_out = f("scale_shift_table").reshape(2, D)
        self.proj_w, self.proj_b = w("proj_out.weight"), f("proj_out.bias")
        # The q RMSNorm weights (self and cross) carry softmax_scale * log2(e):
        # the normed q leaves its norm kernel pre-scaled (still one bf16
        # rounding) and attention starts its scores at -max with no per-score
        # scaling.
        q_mult = ops.LOG2E / math.sqrt(cfg.head_dim)
        self.blocks = []
        for i in range(cfg.layers):
            b = f"blocks.{i}"
            a1, a2 = f"{b}.attn1", f"{b}.attn2"
            blk = {
                "sst": f(f"{b}.scale_shift_table").reshape(6, D),
                "qkv_w": torch.cat([w(f"{a1}.to_q.weight"), w(f"{a1}.to_k.weight"), w(f"{a1}.to_v.weight")]),
                "qkv_b": torch.cat([f(f"{a1}.to_q.bias"), f(f"{a1}.to_k.bias"), f(f"{a1}.to_v.bias")]),
                "nq1_pre": f(f"{a1}.norm_q.weight") * q_mult, "nk1": f(f"{a1}.norm_k.weight"),
                "o1_w": w(f"{a1}.to_out.0.weight"), "o1_b": f(f"{a1}.to_out.0.bias"),
                "n2_w": f(f"{b}.norm2.weight"), "n2_b": f(f"{b}.norm2.bias"),
                "q2_w": w(f"{a2}.to_q.weight"), "q2_b": f(f"{a2}.to_q.bias"),
                "kv2_w": torch.cat([w(f"{a2}.to_k.weight"), w(f"{a2}.to_v.weight")]),
                "kv2_b": torch.cat([f(f"{a2}.to_k.bias"), f(f"{a2}.to_v.bias")]),
                "nq2_pre": f(f"{a2}.norm_q.weight") * q_mult, "nk2": f(f"{a2}.norm_k.weight"),
                "o2_w": w(f"{a2}.to_out.0.weight"), "o2_b": f(f"{a2}.to_out.0.bias"),
                "f1_w": w(f"{b}.ffn.net.0.proj.weight"), "f1_b": f(f"{b}.ffn.net.0.proj.bias"),
                "f2_w": w(f"{b}.ffn.net.2.weight"), "f2_b": f(f"{b}.ffn.net.2.bias"),
            }
            self.blocks.append(blk)
        self.rope_cos, self.rope_sin = rope_tables(cfg.head_dim, cfg.rope_max_seq_len, cfg.rope_theta, dev)
        self.rope_pairs = rope_axis_pairs(cfg.head_dim)
        self.profiler = _NULL_PROFILER

    @classmethod
    def random(cls, cfg, seed=0, device="cuda"):
        return cls(cfg, random_state_dict(cfg, seed, device), device)

    # ------------------------------------------------------------------ prelude
    def _grid(self, latent_shape):
        pt, ph, pw = self.cfg.patch
        _, f, h, w = latent_shape[-4:]
        if f % pt or h % ph or w % pw:
            raise ValueError(f"latent {tuple(latent_shape)} not divisible by patch {self.cfg.patch}")
        return (f // pt, h // ph, w // pw)

    def condition(self, timesteps, texts):
        """Condition embedder over R requests: timesteps [R] fp32 (device),
        texts [R*L, text_dim] bf16 -> temb [R, D] bf16, projected [R, 6, D] fp32,
        encoder [R*L, D] bf16."""
        e = ops.timestep_embedding(timesteps, self.cfg.freq_dim)
        t1 = ops.linear(e, self.te1_w, self.te1_b, "silu")
        temb = ops.linear(t1, self.te2_w, self.te2_b)
        proj = ops.linear(ops.silu(temb), self.tp_w, self.tp_b)
        projected = proj.float().reshape(-1, 6, self.cfg.dim)
        x1 = ops.linear(texts, self.tx1_w, self.tx1_b, "gelu")
        enc = ops.linear(x1, self.tx2_w, self.tx2_b)
        return temb, projected, enc

    def begin_packed_packet(self, latents, timesteps, texts):
        """Packed prelude for R requests.

        latents: list of [C, F, H, W] (any float dtype, device), one per request
        (a CFG pair is two requests sharing a latent); timesteps: list of floats;
        texts: list of [L, text_dim] contexts (zero-padded rows attend)."""
        cfg, dev = self.cfg, self.device
        if not (len(latents) == len(timesteps) == len(texts)) or not latents:
            raise ValueError("latents, timesteps and texts must be non-empty lists of equal length")
        for t in texts:
            if t.dim() < 2 or t.shape[-1] != cfg.text_dim:
                raise ValueError(f"text contexts must be [L, {cfg.text_dim}], got {tuple(t.shape)}")
        for lat in latents:
            if lat.dim() < 4 or lat.shape[-4] != cfg.in_ch:
                raise ValueError(f"latents must be [{cfg.in_ch}, F, H, W], got {tuple(lat.shape)}")
        grids = [self._grid(l.shape) for l in latents]
        counts = [g[0] * g[1] * g[2] for g in grids]
        seg = Segments([0] + [sum(counts[: i + 1]) for i in range(len(counts))], dev)
        hidden = torch.empty((seg.total, cfg.dim), dtype=_BF16, device=dev)
        cache = {}
        for i, lat in enumerate(latents):
            key = (lat.data_ptr(), tuple(lat.shape), tuple(lat.stride()), lat.dtype, lat.device)
            if key in cache:  # CFG pairs share the latent: patchify once
                hidden[seg.cu[i]:seg.cu[i + 1]] = hidden[cache[key][0]:cache[key][1]]
                continue
            patches = ops.patchify(lat.reshape(lat.shape[-4:]).to(_BF16), cfg.patch)
            ops.linear(patches, self.patch_w, self.patch_b, out=hidden[seg.cu[i]:seg.cu[i + 1]])
            cache[key] = (seg.cu[i], seg.cu[i + 1])
        text_lens = [int(t.shape[-2]) for t in texts]
        seg_txt = Segments([0] + [sum(text_lens[: i + 1]) for i in range(len(text_lens))], dev)
        text = torch.cat([t.reshape(-1, cfg.text_dim).to(device=dev, dtype=_BF16) for t in texts])
        t = ops.to_device([float(x) for x in timesteps], torch.float32, dev)
        temb, projected, enc = self.condition(t, text)
        rope = ops.Rope(self.rope_cos, self.rope_sin, grids, seg, self.rope_pairs[0], self.rope_pairs[1])
        packet = dict(hidden=hidden, encoder=enc, temb=temb, projected=projected, rotary=rope,
                      shape=[(1, *g, *cfg.patch) for g in grids], pad_amount=0, local_rows=0, valid_kv_len=None,
                      thw=[list(g) for g in grids], cu_seqlens_q=seg, cu_seqlens_kv_text=seg_txt, grids=grids)
        if len(set(text_lens)) > 1:
            packet["text_lens"] = text_lens
        return packet

    def resolve_packet(self, packet):
        """Rebuild the derived entries of a packet that was carried by a codec
        (workers/ditserve/models/wan/block.py:885-1007): only hidden, encoder, temb,
        projected, rotary (tensors), shape and thw (lists) travel; the segment
        tables, grids and RoPE object follow from them.  Idempotent."""
        if isinstance(packet.get("rotary"), ops.Rope) and "cu_seqlens_q" in packet:
            return packet
        grids = [tuple(int(v) for v in g) for g in packet["thw"]]
        counts = [g[0] * g[1] * g[2] for g in grids]
        seg = Segments([0] + [sum(counts[: i + 1]) for i in range(len(counts))], self.device)
        if seg.total != packet["hidden"].shape[0]:
            raise ValueError("packet grids do not match its hidden rows")
        text_lens = packet.get("text_lens")
        if text_lens is None:
            rows = packet["encoder"].shape[0]
            if rows % len(grids):
                raise ValueError("non-uniform text lengths need the packet's text_lens")
            text_lens = [rows // len(grids)] * len(grids)
        seg_txt = Segments([0] + [sum(text_lens[: i + 1]) for i in range(len(text_lens))], self.device)
        tables = tuple(packet["rotary"])
        if len(tables) != 2:
            raise ValueError("packet rotary must carry the two RoPE angle tables")
        cos, sin = (t.to(device=self.device, dtype=torch.float32).contiguous() for t in tables)
        packet.update(rotary=ops.Rope(cos, sin, grids, seg, self.rope_pairs[0], self.rope_pairs[1]),
                      cu_seqlens_q=seg, cu_seqlens_kv_text=seg_txt, grids=grids)
        return packet

    def begin_packet(self, hidden_states, timestep, encoder_hidden_states):
        """Reference-shaped prelude (transformer_wan.py:307-366) for B requests
        stacked on dim 0: hidden_states [B, C, F, H, W], timestep [B] (or
        [B, S] for Wan2.2 per-token timesteps, all equal per request under the
        all-ones T2V mask of workers/ditserve/models/wan/runtime.py:153-163),
        encoder_hidden_states [B, L, text_dim]."""
        b = hidden_states.shape[0]
        ts = timestep.reshape(b, -1)
        if ts.shape[1] > 1 and not bool((ts == ts[:, :1]).all()):
            raise ValueError("per-token timesteps must be uniform within a request")
        return self.begin_packed_packet([hidden_states[i] for i in range(b)], [float(ts[i, 0]) for i in range(b)],
                                        [encoder_hidden_states[i] for i in range(b)])

    # -------------------------------------------------------------------- block
    def forward_block(self, packet, index):
        """One block over the packed batch; returns and stores the new hidden."""
        cfg, blk, prof = self.cfg, self.blocks[index], self.profiler
        D, H, Dh = cfg.dim, cfg.heads, cfg.head_dim
        self.resolve_packet(packet)
        seg, seg_txt = packet["cu_seqlens_q"], packet["cu_seqlens_kv_text"]
        h = packet["hidden"]
        with prof.region("modulation"):
            mod = ops.modulation(blk["sst"], packet["projected"])  # [R, 6, D] fp32
        # self-attention (_stage1, block.py:282-285)
        with prof.region("adaln"):
            x = ops.adaln(h, mod[:, 0], mod[:, 1], seg, eps=cfg.eps)
        with prof.region("gemm_qkv"):
            qkv = ops.linear(x, blk["qkv_w"], blk["qkv_b"])
        q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
        with prof.region("qk_norm_rope"):
            ops.qk_norm_rope_(q, k, blk["nq1_pre"], blk["nk1"], Dh, cfg.eps, rope=packet["rotary"])
        with prof.region("transpose_v"):
            vt = ops.transpose_v(v, H, Dh, seg)
        with prof.region("attn_self"):
            a = ops.flash_attn_varlen(q, k, None, seg, seg, H, Dh, vt=vt, q_prescaled=True)
        with prof.region("gemm_o_gate"):
            h = ops.linear(a, blk["o1_w"], blk["o1_b"], "gate_res", residual=h, gate=mod[:, 2], segments=seg)
        # cross-attention (_stage2, block.py:288-290)
        with prof.region("cross_prep"):
            x = ops.adaln(h, weight=blk["n2_w"], bias=blk["n2_b"], eps=cfg.eps)
            with prof.region("gemm_cross_q"):
                q2 = ops.linear(x, blk["q2_w"], blk["q2_b"])
            kv2 = ops.linear(packet["encoder"], blk["kv2_w"], blk["kv2_b"])
            k2, v2 = kv2[:, :D], kv2[:, D:]
            # RMSNorm across heads of the image queries and the text keys, in place, one launch
            ops.adaln_multi([dict(x=q2, weight=blk["nq2_pre"], eps=cfg.eps, kind="rms", out=q2),
                             dict(x=k2, weight=blk["nk2"], eps=cfg.eps, kind="rms", out=k2)])
            vt2 = ops.transpose_v(v2, H, Dh, seg_txt)
        with prof.region("attn_cross"):
            a = ops.flash_attn_varlen(q2, k2, None, seg, seg_txt, H, Dh, vt=vt2, q_prescaled=True)
        with prof.region("gemm_o_res"):
            ops.linear(a, blk["o2_w"], blk["o2_b"], "res", residual=h, out=h)
        # FFN (block.py:291-293)
        with prof.region("adaln"):
            x = ops.adaln(h, mod[:, 3], mod[:, 4], seg, eps=cfg.eps)
        with prof.region("gemm_ffn_up_gelu"):
            f = ops.linear(x, blk["f1_w"], blk["f1_b"], "gelu")
        with prof.region("gemm_ffn_down_gate"):
            ops.linear(f, blk["f2_w"], blk["f2_b"], "gate_res", residual=h, gate=mod[:, 5], segments=seg, out=h)
        packet["hidden"] = h
        return h

    # --------------------------------------------------------------- epilogue
    def prediction_packed(self, packet):
        """norm_out AdaLN + proj_out + unpatchify per request -> list of fp32 [C, F, H, W]."""
        cfg = self.cfg
        self.resolve_packet(packet)
        seg = packet["cu_seqlens_q"]
        # (scale_shift_table [2, D] + temb[:, None]) -> shift, scale   (block.py:441-445)
        temb = packet["temb"].float().reshape(-1, 1, cfg.dim).expand(-1, 2, -1)
        mod = ops.modulation(self.sst_out, temb)  # [R, 2, D]
        x = ops.adaln(packet["hidden"], mod[:, 0], mod[:, 1], seg, eps=cfg.eps)
        y = ops.linear(x, self.proj_w, self.proj_b)
        outs = []
        for i, g in enumerate(packet["grids"]):
            outs.append(ops.unpatchify(y[seg.cu[i]:seg.cu[i + 1]], g, cfg.patch, cfg.out_ch))
        return outs

    def prediction(self, packet):
        """Reference-shaped epilogue (transformer_wan.py:378-395): [B, C, F, H, W] fp32."""
        return torch.stack(self.prediction_packed(packet))

    def forward(self, hidden_states, timestep, encoder_hidden_states):
        packet = self.begin_packet(hidden_states, timestep, encoder_hidden_states)
        for i in range(self.cfg.layers):
            self.forward_block(packet, i)
        return self.prediction(packet)

    def forward_packed(self, latents, timesteps, texts):
        packet = self.begin_packed_packet(latents, timesteps, texts)
        for i in range(self.cfg.layers):
            self.forward_block(packet, i)
        return self.prediction_packed(packet)


_SLOT_ROPE = []  # [(weakref cos, weakref sin, cos version, sin version, (device, B, S, dh), Rope)]
_SLOT_ROPE_MAX = 8


def _slot_rope(freqs_cos, freqs_sin, device, B, S, dh):
    """Rotation and segment tables of the slot for these exact table tensors.

    An entry is reused only while the very tensors it was built from are alive and
    unmodified: it holds weak references to them and their version counters, so a
    new table that the caching allocator places at a freed table's address (the
    reference builds fresh tables in every begin_packet, transformer_wan.py:326)
    never matches an old entry."""
    shape = (device, B, S, dh)
    # entries whose tables were freed can never match again: drop them
    _SLOT_ROPE[:] = [e for e in _SLOT_ROPE if e[0]() is not None and e[1]() is not None]
    for e in _SLOT_ROPE:
        if (e[0]() is freqs_cos and e[1]() is freqs_sin and e[2] == freqs_cos._version
                and e[3] == freqs_sin._version and e[4] == shape):
            return e[5]
    # per-token tables: pair i uses cos[..., 2i] / sin[..., 2i+1]
    cos_tab = freqs_cos.reshape(S, dh)[:, 0::2].float().contiguous()
    sin_tab = freqs_sin.reshape(S, dh)[:, 1::2].float().contiguous()
    seg = Segments([b * S for b in range(B + 1)], device)
    rope = ops.Rope(cos_tab, sin_tab, [(S, 1, 1)] * B, seg, dh // 2, 0)
    _SLOT_ROPE.append((weakref.ref(freqs_cos), weakref.ref(freqs_sin), freqs_cos._version, freqs_sin._version,
                       shape, rope))
    del _SLOT_ROPE[:-_SLOT_ROPE_MAX]
    return rope


def _slot_norm(norm, D, query):
    """(fp32 weight [D], eps) of a norm_q / norm_k argument: an RMSNorm module
    (torch.nn.RMSNorm or diffusers' RMSNorm: its `weight`, None without an
    elementwise affine, and its `eps`, which torch.nn.RMSNorm leaves None for
    the input dtype's machine epsilon) or a bare weight tensor (eps 1e-6, the
    Wan attention's norm eps)."""
    if isinstance(norm, torch.Tensor):
        w, eps = norm, 1e-6
    else:
        w, eps = getattr(norm, "weight", None), getattr(norm, "eps", 1e-6)
        if eps is None:
            eps = torch.finfo(query.dtype).eps
    if w is None:
        w = torch.ones(D, device=query.device)
    return w.float().contiguous(), float(eps)


def fused_qk_norm_rope(query, key, norm_q, norm_k, freqs_cos, freqs_sin, heads):
    """Drop-in for the reference's `fused_qk_norm_rope` slot
    (transformer_wan.py:24-25,111-115): query/key [B, S, D] bf16, norm_q/norm_k
    modules or tensors holding the RMSNorm weight, freqs_cos/sin [1, S, 1, Dh]
    fp32 tables (repeat-interleaved, as WanRotaryPosEmbed returns them).
    Returns q, k as [B, S, H, Dh] bf16 (new tensors; inputs untouched).

    One out-of-place kernel launch covers the B requests (each a segment of S
    tokens whose position is its index on a single axis) and writes the new
    tensors directly.  The rotation and segment tables built from freqs_cos/sin
    are kept while those same table tensors live unmodified (the 30 blocks of one
    packet pass the same tables), so a steady call allocates only the two outputs."""
    B, S, D = query.shape
    dh = D // heads
    wq, eps_q = _slot_norm(norm_q, D, query)
    wk, eps_k = _slot_norm(norm_k, D, query)
    if eps_q != eps_k:
        raise ValueError(f"norm_q and norm_k must share eps (got {eps_q} and {eps_k})")
    rope = _slot_rope(freqs_cos, freqs_sin, query.device, B, S, dh)
    qi, ki = query.reshape(B * S, D), key.reshape(B * S, D)
    if qi.dtype != _BF16 or qi.stride(1) != 1:
        qi = qi.to(_BF16).contiguous()
    if ki.dtype != _BF16 or ki.stride(1) != 1:
        ki = ki.to(_BF16).contiguous()
    q = torch.empty((B * S, D), dtype=_BF16, device=query.device)
    k = torch.empty((B * S, D), dtype=_BF16, device=query.device)
    ops.qk_norm_rope_(qi, ki, wq, wk, dh, eps_q, rope=rope, out=(q, k))
    return q.reshape(B, S, heads, dh), k.reshape(B, S, heads, dh)


def step_flops(cfg, tokens_per_request, text_len=512):
    """Algorithmic FLOPs of the 30-block transformer over the given requests
    (attention 4*S^2*D per request, GEMMs 2*M*N*K)."""
    total = 0
    D, F = cfg.dim, cfg.ffn
    for s in tokens_per_request:
        per_block = (2 * s * D * 3 * D + 2 * s * D * D * 2 + 2 * text_len * D * 2 * D + 4 * s * s * D
                     + 4 * s * text_len * D + 4 * s * D * F)
        total += per_block * cfg.layers
    return total


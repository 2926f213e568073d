"""Wan at full working-set sizes on the GPU.

* Wan2.1-T2V-1.3B architecture, 30 blocks, latent 16x21x60x104 (480x832x81
  frames): the CFG pair packed as 2 x 32760 tokens, each segment bitwise equal to
  its solo forward.
* Wan2.2-TI2V-5B architecture, 30 blocks, latent 48x31x44x80 (704x1280x121 frames):
  the CFG pair packed as 2 x 27280 tokens (text valid 150 / 0, t = 700) gives finite
  outputs, each segment bitwise equal to its solo forward.
* Two blocks of the Wan2.1-T2V-14B architecture over its 720x1280x81 CFG pair (2 x
  75600 tokens, a 4.6 GB fused QKV buffer), packed bitwise equal to solo; that
  pair's self-attention with q rows past 4 GiB of offsets, on sampled rows against
  an fp32 reference.
* The full Wan2.1-1.3B CFG-pair steps at 480x832x81, 720x1280x81 and 480x832x33
  (2 x 32760, 75600 and 14040 tokens), the Wan2.2-5B 704x1280x121 step (2 x 27280)
  and the 4-request packed batch (56400 tokens), 30 blocks each, against the oracle
  run in fp32 on the GPU: cos >= 0.999 and relative L2 <= 2e-2 per prediction.
* One Wan2.2-5B block at 4096 tokens, one Wan2.1-14B block at 128 tokens and one
  Wan2.1 block at the full 21x30x52 grid (32760 tokens) against the CPU fp32
  oracle (torch's CPU flash SDPA for the 32760-token self-attention), cos >= 0.999
  and relative L2 <= 1e-2.
"""
import math

import pytest
import torch

from oracle import common as oc
from oracle import wan as ow
from tests.helpers import assert_close, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _text(seed, valid, dim=4096, length=512):
    t = randn((length, dim), seed)
    t[valid:] = 0
    return t


def test_wan22_5b_30_blocks_full_latent_cfg_pair_bitwise():
    from ditserve_amd.wan import WAN22_TI2V_5B, WanTransformer
    model = WanTransformer.random(WAN22_TI2V_5B, seed=8, device=DEV)
    lat = randn((48, 31, 44, 80), 50).to(DEV)
    tc, tu = _text(51, 150).to(DEV), torch.zeros(512, 4096, device=DEV)
    packet = model.begin_packed_packet([lat, lat], [700.0, 700.0], [tc, tu])
    assert packet["cu_seqlens_q"].cu == [0, 27280, 54560]
    both = model.forward_packed([lat, lat], [700.0, 700.0], [tc, tu])
    for out, txt in zip(both, (tc, tu)):
        assert out.shape == (48, 31, 44, 80) and bool(torch.isfinite(out).all())
        solo = model.forward_packed([lat], [700.0], [txt])[0]
        assert torch.equal(out, solo)
    assert not torch.equal(both[0], both[1])


def test_wan21_30_blocks_480p_cfg_pair_bitwise():
    """The headline workload's shape: Wan2.1-1.3B architecture, 30 blocks, latent
    16x21x60x104 (480x832x81 frames), the CFG pair packed as 2 x 32760 tokens (text
    valid 120 / 0, t = 999): each segment of the packed forward equals, bitwise,
    the forward of that request alone."""
    from ditserve_amd.wan import WAN21_T2V_1_3B, WanTransformer
    model = WanTransformer.random(WAN21_T2V_1_3B, seed=9, device=DEV)
    lat = randn((16, 21, 60, 104), 52).to(DEV)
    tc, tu = _text(53, 120).to(DEV), torch.zeros(512, 4096, device=DEV)
    packet = model.begin_packed_packet([lat, lat], [999.0, 999.0], [tc, tu])
    assert packet["cu_seqlens_q"].cu == [0, 32760, 65520]
    both = model.forward_packed([lat, lat], [999.0, 999.0], [tc, tu])
    for out, txt in zip(both, (tc, tu)):
        assert out.shape == (16, 21, 60, 104) and bool(torch.isfinite(out).all())
        assert torch.equal(out, model.forward_packed([lat], [999.0], [txt])[0])
    assert not torch.equal(both[0], both[1])


def test_wan21_480p_full_step_matches_oracle():
    """The headline step at its full size against the oracle: Wan2.1-1.3B
    architecture, 30 blocks, latent 16x21x60x104 (480x832x81 frames), the CFG pair
    packed as 2 x 32760 tokens (text valid 120 / 0, t = 999).  The oracle runs in
    fp32 on the GPU, its attention through torch's fp32 memory-efficient SDPA
    (checked first against a float64 softmax on sampled rows at this shape).  Each
    prediction: cosine >= 0.999 and relative L2 <= 2e-2 over the whole step."""
    from ditserve_amd.wan import WAN21_T2V_1_3B, WanTransformer, random_state_dict
    cfg, S = WAN21_T2V_1_3B, 32760
    g = torch.Generator(device=DEV).manual_seed(12)
    q, k, v = (torch.randn((cfg.heads, S, cfg.head_dim), generator=g, device=DEV) for _ in range(3))
    rows = torch.arange(0, S, 4095, device=DEV)
    ref = torch.softmax(q[:, rows].double() @ k.double().transpose(1, 2) / math.sqrt(cfg.head_dim), -1) @ v.double()
    err = ((oc.sdpa_fast(q, k, v)[:, rows].double() - ref).norm() / ref.norm()).item()
    assert err < 1e-5, f"fp32 SDPA relative error {err}"
    del q, k, v, ref
    sd = random_state_dict(cfg, seed=13, device=DEV)
    model = WanTransformer(cfg, sd, DEV)
    lat = randn((16, 21, 60, 104), 56).to(DEV)
    texts = (_text(57, 120).to(DEV), torch.zeros(512, 4096, device=DEV))
    got = [o.float().cpu() for o in model.forward_packed([lat, lat], [999.0, 999.0], list(texts))]
    del model
    torch.cuda.empty_cache()
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    with torch.no_grad():
        for out, txt, label in zip(got, texts, ("cond", "uncond")):
            ref = ow.forward(sd, ocfg, lat.bfloat16().float(), 999.0, txt.bfloat16().float(), attn=oc.sdpa_fast)
            c, r = assert_close(out, ref.cpu(), 0.999, 2e-2, f"wan2.1 480p 30-block step ({label})")
            print(f"{label}: cos {c:.6f} relL2 {r:.3e}")
            del ref


@pytest.mark.parametrize("latent,label", [((16, 21, 90, 160), "720x1280x81, 2 x 75600 tokens"),
                                          ((16, 9, 60, 104), "480x832x33, 2 x 14040 tokens")])
def test_wan21_other_sizes_full_step_matches_oracle(latent, label):
    """The Wan2.1-1.3B CFG-pair step at the reference's other published sizes, 30 blocks
    (text valid 120 / 0, t = 999), against the oracle run in fp32 on the GPU: each
    prediction within cos >= 0.999 and relative L2 <= 2e-2."""
    from ditserve_amd.wan import WAN21_T2V_1_3B, WanTransformer, random_state_dict
    cfg = WAN21_T2V_1_3B
    sd = random_state_dict(cfg, seed=17, device=DEV)
    model = WanTransformer(cfg, sd, DEV)
    lat = randn(latent, 62).to(DEV)
    texts = (_text(63, 120).to(DEV), torch.zeros(512, 4096, device=DEV))
    got = [o.float().cpu() for o in model.forward_packed([lat, lat], [999.0, 999.0], list(texts))]
    del model
    torch.cuda.empty_cache()
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    with torch.no_grad():
        for out, txt, branch in zip(got, texts, ("cond", "uncond")):
            ref = ow.forward(sd, ocfg, lat.bfloat16().float(), 999.0, txt.bfloat16().float(), attn=oc.sdpa_fast)
            c, r = assert_close(out, ref.cpu(), 0.999, 2e-2, f"wan2.1 {label} ({branch})")
            print(f"{label} {branch}: cos {c:.6f} relL2 {r:.3e}")
            del ref


def test_wan22_5b_full_step_matches_oracle():
    """The Wan2.2-TI2V-5B step at its full size (30 blocks, latent 48x31x44x80 for
    704x1280x121 frames, the CFG pair packed as 2 x 27280 tokens, text valid 150 /
    0, t = 700) against the oracle run in fp32 on the GPU: each prediction within
    cos >= 0.999 and relative L2 <= 2e-2."""
    from ditserve_amd.wan import WAN22_TI2V_5B, WanTransformer, random_state_dict
    cfg = WAN22_TI2V_5B
    sd = random_state_dict(cfg, seed=14, device=DEV)
    model = WanTransformer(cfg, sd, DEV)
    lat = randn((48, 31, 44, 80), 58).to(DEV)
    texts = (_text(59, 150).to(DEV), torch.zeros(512, 4096, device=DEV))
    got = [o.float().cpu() for o in model.forward_packed([lat, lat], [700.0, 700.0], list(texts))]
    del model
    torch.cuda.empty_cache()
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    with torch.no_grad():
        for out, txt, label in zip(got, texts, ("cond", "uncond")):
            ref = ow.forward(sd, ocfg, lat.bfloat16().float(), 700.0, txt.bfloat16().float(), attn=oc.sdpa_fast)
            c, r = assert_close(out, ref.cpu(), 0.999, 2e-2, f"wan2.2-5b 704p 30-block step ({label})")
            print(f"{label}: cos {c:.6f} relL2 {r:.3e}")
            del ref


def test_wan_packed_batch_config2_full_size_matches_oracle():
    """The 4-request packed batch at full size (latents 21x60x104, 9x60x104, 13x40x64
    and 5x32x32: 32760 + 14040 + 8320 + 1280 = 56400 tokens; timesteps drawn in
    [0, 1000), texts with 30-200 valid rows), 30 blocks: each request's packed
    prediction against the oracle run in fp32 on the GPU, cos >= 0.999 and relative
    L2 <= 2e-2."""
    from ditserve_amd.wan import WAN21_T2V_1_3B, WanTransformer, random_state_dict
    cfg = WAN21_T2V_1_3B
    sd = random_state_dict(cfg, seed=15, device=DEV)
    model = WanTransformer(cfg, sd, DEV)
    g = torch.Generator().manual_seed(16)
    shapes = [(16, 21, 60, 104), (16, 9, 60, 104), (16, 13, 40, 64), (16, 5, 32, 32)]
    lats = [torch.randn(s, generator=g).to(DEV) for s in shapes]
    ts = [float(x) for x in (torch.rand(4, generator=g) * 1000)]
    valid = [int(x) for x in torch.randint(30, 201, (4,), generator=g)]
    texts = [_text(60 + i, valid[i]).to(DEV) for i in range(4)]
    got = [o.float().cpu() for o in model.forward_packed(lats, ts, texts)]
    del model
    torch.cuda.empty_cache()
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    with torch.no_grad():
        for i, out in enumerate(got):
            ref = ow.forward(sd, ocfg, lats[i].bfloat16().float(), ts[i], texts[i].bfloat16().float(),
                             attn=oc.sdpa_fast)
            c, r = assert_close(out, ref.cpu(), 0.999, 2e-2, f"packed request {i} {shapes[i]} t={ts[i]:.1f}")
            print(f"request {i} {shapes[i]}: cos {c:.6f} relL2 {r:.3e}")
            del ref


def test_wan21_14b_two_blocks_720p_cfg_pair_bitwise():
    """Two blocks of the Wan2.1-T2V-14B architecture (hidden 5120, 40 heads, FFN
    13824) over the 720x1280x81 CFG pair packed as 2 x 75600 tokens: the fused QKV
    buffer (15360 wide) holds 4.6 GB, the GEMMs run K = 5120 and 13824 at
    M = 151200.  Each segment is bitwise its solo forward."""
    import dataclasses

    from ditserve_amd.wan import WAN21_T2V_14B, WanTransformer
    model = WanTransformer.random(dataclasses.replace(WAN21_T2V_14B, layers=2), seed=11, device=DEV)
    lat = randn((16, 21, 90, 160), 54).to(DEV)
    tc, tu = _text(55, 120).to(DEV), torch.zeros(512, 4096, device=DEV)
    both = model.forward_packed([lat, lat], [999.0, 999.0], [tc, tu])
    for out, txt in zip(both, (tc, tu)):
        assert out.shape == (16, 21, 90, 160) and bool(torch.isfinite(out).all())
        assert torch.equal(out, model.forward_packed([lat], [999.0], [txt])[0])
    assert not torch.equal(both[0], both[1])


def test_attention_q_rows_past_4gib():
    """Self-attention of a Wan2.1-14B CFG pair at 720x1280x81 (2 x 75600 tokens, 40
    heads of 128) with q, k, v as column slices of one fused [151200, 3 x 5120] bf16
    QKV buffer: q's rows span 4.6 GB, so rows near the end lie past 4 GiB of byte
    offsets.  Sampled rows (heads 0 and 39; the first rows of segment 0, the last of
    segment 1) against an fp32 reference, through the plain entry point and, after q
    is scaled in place, the pre-scaled one."""
    from ditserve_amd import ops
    H, Dh, S = 40, 128, 75600
    D, T = H * Dh, 2 * S
    g = torch.Generator(device=DEV).manual_seed(5)
    qkv = torch.empty((T, 3 * D), dtype=torch.bfloat16, device=DEV)
    for i in range(0, T, 8192):
        n = min(8192, T - i)
        qkv[i:i + n] = torch.randn((n, 3 * D), generator=g, device=DEV).bfloat16()
    q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    assert (T - 1) * q.stride(0) * 2 >= 2 ** 32
    seg = ops.Segments([0, S, T], DEV)
    rows = {0: torch.arange(0, 48, device=DEV), 1: torch.arange(T - 48, T, device=DEV)}
    refs = {}
    for m, r in rows.items():
        for h in (0, H - 1):
            cols = slice(h * Dh, (h + 1) * Dh)
            kk, vv = k[m * S:(m + 1) * S, cols].float(), v[m * S:(m + 1) * S, cols].float()
            p = torch.softmax(q[r, cols].float() @ kk.t() / math.sqrt(Dh), dim=-1)
            refs[(m, h)] = p @ vv
    out = ops.flash_attn_varlen(q, k, v, seg, seg, H, Dh)
    for (m, h), ref in refs.items():
        assert_close(out[rows[m], h * Dh:(h + 1) * Dh].float().cpu(), ref.cpu(), 0.9999, 1e-2, f"plain seg {m} head {h}")
    del out
    qkv[:, :D] = (q.float() * (ops.LOG2E / math.sqrt(Dh))).bfloat16()
    vt = ops.transpose_v(v, H, Dh, seg)
    out = ops.flash_attn_varlen(q, k, None, seg, seg, H, Dh, vt=vt, q_prescaled=True)
    for (m, h), ref in refs.items():
        # q rounded to bf16 once more after the scaling: a looser bound
        assert_close(out[rows[m], h * Dh:(h + 1) * Dh].float().cpu(), ref.cpu(), 0.999, 2e-2, f"pre seg {m} head {h}")


def _block_vs_oracle(cfg, grid, text_valid, t, seed, attn, label):
    from ditserve_amd.wan import WanTransformer, random_state_dict
    sd = random_state_dict(cfg, seed=seed)
    model = WanTransformer(cfg, sd, DEV)
    f, h, w = grid
    lat = randn((cfg.in_ch, f, 2 * h, 2 * w), seed + 1)
    packet = model.begin_packed_packet([lat.to(DEV)], [t], [_text(seed + 2, text_valid).to(DEV)])
    h_in, e_in, p_in = packet["hidden"].float().cpu(), packet["encoder"].float().cpu(), packet["projected"][0].cpu()
    out = model.forward_block(packet, 0).float().cpu()
    del model, packet
    torch.cuda.empty_cache()
    cos, sin = ow.rope_freqs(grid)
    ref = ow.block_forward(sd, 0, h_in, e_in, p_in, cos, sin, cfg.heads, attn=attn)
    assert_close(out, ref, 0.999, 1e-2, label)


def test_wan22_5b_block_4096_tokens_matches_oracle():
    from ditserve_amd.wan import WanConfig
    cfg = WanConfig(dim=3072, heads=24, ffn=14336, in_ch=48, out_ch=48, layers=1)
    _block_vs_oracle(cfg, (4, 32, 32), 150, 700.0, 60, oc.sdpa, "wan2.2-5b block, 4096 tokens")


def test_wan21_14b_block_matches_oracle():
    """One block of the Wan2.1-T2V-14B architecture (D = 5120, 40 heads, FFN 13824:
    the widest rows the row kernels take, 10 chunks per lane) over 128 tokens."""
    from ditserve_amd.wan import WAN21_T2V_14B
    import dataclasses
    cfg = dataclasses.replace(WAN21_T2V_14B, layers=1)
    _block_vs_oracle(cfg, (2, 8, 8), 77, 500.0, 80, oc.sdpa, "wan2.1-14b block, 128 tokens")


def test_wan21_block_full_grid_32760_tokens_matches_oracle():
    from ditserve_amd.wan import WanConfig
    _block_vs_oracle(WanConfig(layers=1), (21, 30, 52), 120, 999.0, 70, oc.sdpa_fast,
                     "wan2.1 block, 32760 tokens")

"""Wan transformer on the GPU against the CPU fp32 oracle.

Tolerances (north star): per block cos >= 0.999 and relative L2 <= 1e-2; a full
30-block step relative L2 <= 2e-2; packed execution bitwise equal to
per-request runs.  Weights are seeded random-init (see random_state_dict)."""
import pytest
import torch

from oracle import wan as ow
from tests.helpers import assert_close, bf, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _wan():
    from ditserve_amd import wan
    return wan


def _text(seed, valid, dim=4096, length=512):
    t = randn((length, dim), seed)
    t[valid:] = 0
    return t


def test_wan21_block_config0_matches_oracle():
    """One Wan2.1-1.3B block, 1x30x52 grid (1560 tokens), 512 text tokens (77 valid), t=500."""
    wan = _wan()
    cfg = wan.WanConfig(layers=1)
    sd = wan.random_state_dict(cfg, seed=0)
    model = wan.WanTransformer(cfg, sd, DEV)
    lat, text = randn((16, 1, 60, 104), 1), _text(2, 77)
    packet = model.begin_packed_packet([lat.to(DEV)], [500.0], [text.to(DEV)])
    # prelude: patch embedding + condition embedder
    assert_close(packet["hidden"].float().cpu(), ow.patch_embed(sd, bf(lat)), 0.99999, 5e-3, "patch_embed")
    temb, proj, enc = ow.condition_embedder(sd, torch.tensor([500.0]), bf(text))
    assert_close(packet["temb"].float().cpu(), temb, 0.9999, 1e-2, "temb")
    assert_close(packet["projected"].cpu(), proj, 0.9999, 1e-2, "projected")
    assert_close(packet["encoder"].float().cpu(), enc, 0.9999, 1e-2, "encoder")
    # block on identical inputs
    h_in, e_in, p_in = packet["hidden"].float().cpu(), packet["encoder"].float().cpu(), packet["projected"][0].cpu()
    out = model.forward_block(packet, 0).float().cpu()
    cos, sin = ow.rope_freqs((1, 30, 52))
    ref = ow.block_forward(sd, 0, h_in, e_in, p_in, cos, sin, cfg.heads)
    assert_close(out, ref, 0.999, 1e-2, "wan2.1 block")


def test_wan21_full_step_30_blocks_matches_oracle():
    """Full 30-block Wan2.1-1.3B forward (prelude, blocks, prediction) on a 2x8x16 grid."""
    wan = _wan()
    cfg = wan.WAN21_T2V_1_3B
    sd_dev = wan.random_state_dict(cfg, seed=1, device=DEV)
    model = wan.WanTransformer(cfg, sd_dev, DEV)
    sd = {k: v.cpu() for k, v in sd_dev.items()}
    del sd_dev
    lat, text = randn((16, 2, 16, 32), 3), _text(4, 120)
    got = model.forward_packed([lat.to(DEV)], [999.0], [text.to(DEV)])[0].cpu()
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    ref = ow.forward(sd, ocfg, bf(lat), 999.0, bf(text))
    assert_close(got, ref, 0.999, 2e-2, "wan2.1 30-block step")


def test_wan22_5b_block_matches_oracle():
    """One Wan2.2-TI2V-5B-architecture block (dim 3072, 24 heads, FFN 14336)."""
    wan = _wan()
    cfg = wan.WanConfig(dim=3072, heads=24, ffn=14336, in_ch=48, out_ch=48, layers=1)
    sd = wan.random_state_dict(cfg, seed=2)
    model = wan.WanTransformer(cfg, sd, DEV)
    lat, text = randn((48, 3, 16, 20), 5), _text(6, 150)
    packet = model.begin_packed_packet([lat.to(DEV)], [700.0], [text.to(DEV)])
    h_in, e_in, p_in = packet["hidden"].float().cpu(), packet["encoder"].float().cpu(), packet["projected"][0].cpu()
    out = model.forward_block(packet, 0).float().cpu()
    cos, sin = ow.rope_freqs((3, 8, 10))
    ref = ow.block_forward(sd, 0, h_in, e_in, p_in, cos, sin, cfg.heads)
    assert_close(out, ref, 0.999, 1e-2, "wan2.2 block")


def test_wan22_per_token_timesteps_equal_per_request():
    """Wan2.2 TI2V passes one timestep per patch token (all equal under the T2V mask,
    workers/ditserve/models/wan/runtime.py:153-163); begin_packet accepts [B, S] and
    gives the same packet as the per-request timestep."""
    wan = _wan()
    cfg = wan.WanConfig(dim=256, heads=2, ffn=512, layers=1, in_ch=48, out_ch=48, text_dim=64)
    model = wan.WanTransformer.random(cfg, seed=3, device=DEV)
    lat = randn((1, 48, 3, 8, 8), 7).to(DEV)
    text = randn((1, 16, 64), 8).to(DEV)
    ts = ow.model_timestep(lat.shape, 700.0, True).to(DEV)
    a = model.begin_packet(lat, ts, text)
    b = model.begin_packet(lat, torch.tensor([700.0], device=DEV), text)
    assert torch.equal(a["projected"], b["projected"]) and torch.equal(a["hidden"], b["hidden"])
    with pytest.raises(ValueError):
        ts2 = ts.clone()
        ts2[0, 3] = 1.0
        model.begin_packet(lat, ts2, text)


def test_wan_packed_batch_config2_bitwise_equals_solo():
    """4 requests (21x30x52, 9x30x52, 13x20x32, 5x16x16 grids = 56400 tokens), own
    timesteps and texts, 30 blocks: each request's packed output == its solo run, bitwise."""
    wan = _wan()
    cfg = wan.WAN21_T2V_1_3B
    model = wan.WanTransformer.random(cfg, seed=4, device=DEV)
    g = torch.Generator().manual_seed(5)
    shapes = [(16, 21, 60, 104), (16, 9, 60, 104), (16, 13, 40, 64), (16, 5, 32, 32)]
    lats = [torch.randn(s, generator=g).to(DEV) for s in shapes]
    ts = [float(x) for x in (torch.rand(4, generator=g) * 1000)]
    valid = [int(x) for x in torch.randint(30, 201, (4,), generator=g)]
    texts = [_text(10 + i, valid[i]).to(DEV) for i in range(4)]
    packet = model.begin_packed_packet(lats, ts, texts)
    assert packet["cu_seqlens_q"].cu == [0, 32760, 46800, 55120, 56400]
    assert packet["cu_seqlens_kv_text"].cu == [0, 512, 1024, 1536, 2048]
    packed = model.forward_packed(lats, ts, texts)
    for i in range(4):
        solo = model.forward_packed([lats[i]], [ts[i]], [texts[i]])[0]
        assert torch.isfinite(solo).all()
        assert torch.equal(packed[i], solo), f"request {i} differs"


def test_cfg_pair_packing_bitwise():
    """A CFG pair (cond, uncond) packed as two segments equals two separate forwards."""
    wan = _wan()
    cfg = wan.WanConfig(layers=2)
    model = wan.WanTransformer.random(cfg, seed=6, device=DEV)
    lat = randn((16, 3, 20, 24), 20).to(DEV)
    tc, tu = _text(21, 120).to(DEV), torch.zeros(512, 4096, device=DEV)
    both = model.forward_packed([lat, lat], [999.0, 999.0], [tc, tu])
    assert torch.equal(both[0], model.forward_packed([lat], [999.0], [tc])[0])
    assert torch.equal(both[1], model.forward_packed([lat], [999.0], [tu])[0])


def test_fused_qk_norm_rope_slot():
    """The reference slot signature (query/key [B,S,D], norm modules, freqs [1,S,1,Dh]):
    two requests in one call, each equal to the oracle; a second call (cached
    tables) gives the same bits and the inputs stay untouched."""
    wan = _wan()
    B, S, D, H = 2, 300, 1536, 12
    grid = (3, 10, 10)
    q, k = bf(randn((B, S, D), 30)), bf(randn((B, S, D), 31))
    wq, wk = bf(randn((D,), 32, 0.1) + 1), bf(randn((D,), 33, 0.1) + 1)
    cos, sin = ow.rope_freqs(grid)
    qd, kd = q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16)
    args = (wq.to(DEV), wk.to(DEV), cos.reshape(1, S, 1, 128).to(DEV), sin.reshape(1, S, 1, 128).to(DEV), H)
    oq, okk = wan.fused_qk_norm_rope(qd, kd, *args)
    assert oq.shape == (B, S, H, 128) and okk.shape == (B, S, H, 128)
    for b in range(B):
        rq, rk = ow.qk_norm_rope(q[b], k[b], wq, wk, cos, sin, H)
        assert_close(oq[b].float().cpu(), rq, 0.99999, 5e-3, f"slot q[{b}]")
        assert_close(okk[b].float().cpu(), rk, 0.99999, 5e-3, f"slot k[{b}]")
    oq2, okk2 = wan.fused_qk_norm_rope(qd, kd, *args)
    assert torch.equal(oq2, oq) and torch.equal(okk2, okk)
    assert torch.equal(qd.cpu(), q.to(torch.bfloat16)) and torch.equal(kd.cpu(), k.to(torch.bfloat16))


def test_fused_qk_norm_rope_slot_norm_modules():
    """norm_q / norm_k passed as torch.nn.RMSNorm modules, as the reference's
    processor passes attn.norm_q / attn.norm_k: their weights and eps (here 1e-5)
    are the ones applied."""
    wan = _wan()
    B, S, D, H = 1, 300, 1536, 12
    grid = (3, 10, 10)
    q, k = bf(randn((B, S, D), 38)) * 1e-3, bf(randn((B, S, D), 39)) * 1e-3
    q, k = bf(q), bf(k)
    wq, wk = bf(randn((D,), 40, 0.1) + 1), bf(randn((D,), 41, 0.1) + 1)
    mods = []
    for w in (wq, wk):
        m = torch.nn.RMSNorm(D, eps=1e-5).to(DEV)
        with torch.no_grad():
            m.weight.copy_(w)
        mods.append(m)
    cos, sin = ow.rope_freqs(grid)
    oq, okk = wan.fused_qk_norm_rope(q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16), *mods,
                                     cos.reshape(1, S, 1, 128).to(DEV), sin.reshape(1, S, 1, 128).to(DEV), H)
    rq, rk = ow.qk_norm_rope(q[0], k[0], wq, wk, cos, sin, H, eps=1e-5)
    assert_close(oq[0].float().cpu(), rq, 0.99999, 5e-3, "slot q, module norms")
    assert_close(okk[0].float().cpu(), rk, 0.99999, 5e-3, "slot k, module norms")
    # rows of mean square ~1e-6 tell eps 1e-5 from 1e-6: the oracle at 1e-6 is far off
    wrong, _ = ow.qk_norm_rope(q[0], k[0], wq, wk, cos, sin, H, eps=1e-6)
    assert (oq[0].float().cpu() - wrong).norm() > 0.1 * wrong.norm()


def test_fused_qk_norm_rope_slot_fresh_tables_of_equal_length():
    """Two packets of equal S but different grids, (2, 6, 25) then (2, 10, 15): the
    first packet's tables are freed before the second packet builds its own (as the
    reference does per begin_packet, transformer_wan.py:326), so the caching
    allocator may place them at the same address.  Each call must rotate with its
    own tables."""
    wan = _wan()
    B, S, D, H = 1, 300, 1536, 12
    q, k = bf(randn((B, S, D), 34)), bf(randn((B, S, D), 35))
    wq, wk = bf(randn((D,), 36, 0.1) + 1), bf(randn((D,), 37, 0.1) + 1)
    qd, kd = q.to(DEV, torch.bfloat16), k.to(DEV, torch.bfloat16)
    ptrs = []
    for grid in ((2, 6, 25), (2, 10, 15)):
        cos, sin = ow.rope_freqs(grid)
        cd, sd = cos.reshape(1, S, 1, 128).to(DEV), sin.reshape(1, S, 1, 128).to(DEV)
        ptrs.append(cd.data_ptr())
        oq, okk = wan.fused_qk_norm_rope(qd, kd, wq.to(DEV), wk.to(DEV), cd, sd, H)
        rq, rk = ow.qk_norm_rope(q[0], k[0], wq, wk, cos, sin, H)
        assert_close(oq[0].float().cpu(), rq, 0.99999, 5e-3, f"slot q {grid}")
        assert_close(okk[0].float().cpu(), rk, 0.99999, 5e-3, f"slot k {grid}")
        del cd, sd, oq, okk
    print("table addresses", [hex(p) for p in ptrs], "reused" if ptrs[0] == ptrs[1] else "distinct")

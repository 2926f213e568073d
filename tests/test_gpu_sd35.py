"""SD3.5-Medium MMDiT on the GPU against the CPU fp32 oracle, and packed vs solo.

Tolerances: a multi-block forward within cos >= 0.999 and relative L2 <= 2e-2 of
the oracle (the north star's full-step bound); packed segments bitwise equal to
solo runs; cu_seqlens bit-exact."""
import json
import os

import pytest
import torch

from oracle import sd35 as osd
from tests.helpers import assert_close, bf, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "packing_vectors.json")))


def _sd():
    from ditserve_amd import sd35
    return sd35


def _inputs(seed, res, n_txt=333):
    lat = randn((16, res // 8, res // 8), seed)
    txt = randn((n_txt, 4096), seed + 1)
    pooled = randn((2048,), seed + 2)
    return lat, txt, pooled


def test_sd35_small_depth_packed_matches_oracle_and_solo():
    """3 blocks (dual attention in block 0, context_pre_only block 2), two requests of
    different resolutions and timesteps packed together."""
    sd35 = _sd()
    cfg = sd35.SD35Config(layers=3, dual_layers=(0,))
    sd = sd35.random_state_dict(cfg, seed=0)
    model = sd35.SD35Transformer(cfg, sd, DEV)
    reqs = [_inputs(1, 256), _inputs(5, 128)]
    ts = [500.0, 37.0]
    outs, meta = model.forward_packed([r[0].to(DEV) for r in reqs], ts, [r[1].to(DEV) for r in reqs],
                                      [r[2].to(DEV) for r in reqs])
    assert meta["cu_seqlens_img"] == [0, 256, 320] and meta["cu_seqlens_joint"] == [0, 589, 986]
    for m, (lat, txt, pooled) in enumerate(reqs):
        ref = osd.forward(sd, cfg.oracle_dict(), bf(lat), ts[m], bf(txt), bf(pooled))
        assert_close(outs[m].cpu(), ref, 0.999, 2e-2, f"sd35 3-block request {m}")
        solo, _ = model.forward_packed([lat.to(DEV)], [ts[m]], [txt.to(DEV)], [pooled.to(DEV)])
        assert torch.equal(outs[m], solo[0]), f"request {m}: packed != solo"


def test_sd35_non_square_packed_matches_oracle_and_solo():
    """Non-square requests packed together: 1024 x 576 and 512 x 768 pixels (64 x 36 and
    32 x 48 patches), 3 blocks (dual attention in block 0, context_pre_only block 2),
    own timesteps and prompt lengths (333 and 154 text tokens): each against the oracle
    and bitwise equal to its solo run (the position crop, patchify and unpatchify keep
    rows and columns apart; the joint seams sit at different offsets)."""
    sd35 = _sd()
    cfg = sd35.SD35Config(layers=3, dual_layers=(0,))
    sd = sd35.random_state_dict(cfg, seed=6)
    model = sd35.SD35Transformer(cfg, sd, DEV)
    lats = [randn((16, 128, 72), 70), randn((16, 64, 96), 71)]
    txts, pools = [randn((333, 4096), 72), randn((154, 4096), 73)], [randn((2048,), 74), randn((2048,), 75)]
    ts = [640.0, 120.0]
    outs, meta = model.forward_packed([x.to(DEV) for x in lats], ts, [x.to(DEV) for x in txts],
                                      [x.to(DEV) for x in pools])
    assert meta["cu_seqlens_img"] == [0, 2304, 3840] and meta["cu_seqlens_txt"] == [0, 333, 487]
    assert meta["cu_seqlens_joint"] == [0, 2637, 4327]
    for m in range(2):
        assert outs[m].shape == lats[m].shape
        ref = osd.forward(sd, cfg.oracle_dict(), bf(lats[m]), ts[m], bf(txts[m]), bf(pools[m]))
        assert_close(outs[m].cpu(), ref, 0.999, 2e-2, f"sd35 non-square request {m}")
        solo, _ = model.forward_packed([lats[m].to(DEV)], [ts[m]], [txts[m].to(DEV)], [pools[m].to(DEV)])
        assert torch.equal(outs[m], solo[0]), f"request {m}: packed != solo"


def test_sd35_large_shaped_blocks_match_oracle():
    """The SD3.5-Large block shape (38 heads of 64, hidden 2432, FFN 9728, no dual
    attention, position table 192), two blocks (the second context_pre_only) at 256^2."""
    sd35 = _sd()
    cfg = sd35.SD35Config(dim=2432, heads=38, layers=2, dual_layers=(), ffn=9728, pos_max=192)
    sd = sd35.random_state_dict(cfg, seed=3)
    model = sd35.SD35Transformer(cfg, sd, DEV)
    lat, txt, pooled = _inputs(20, 256)
    outs, _ = model.forward_packed([lat.to(DEV)], [400.0], [txt.to(DEV)], [pooled.to(DEV)])
    ref = osd.forward(sd, cfg.oracle_dict(), bf(lat), 400.0, bf(txt), bf(pooled))
    assert_close(outs[0].cpu(), ref, 0.999, 2e-2, "sd35-large-shaped 2 blocks")


def test_sd35_medium_24_blocks_512px_matches_oracle():
    """Full SD3.5-Medium architecture (24 joint blocks, 13 dual) at 512^2 (1024 image tokens)."""
    sd35 = _sd()
    cfg = sd35.SD35_MEDIUM
    sd_dev = sd35.random_state_dict(cfg, seed=1, device=DEV)
    model = sd35.SD35Transformer(cfg, sd_dev, DEV)
    sd = {k: v.cpu() for k, v in sd_dev.items()}
    del sd_dev
    lat, txt, pooled = _inputs(10, 512)
    out = model.forward(lat.unsqueeze(0).to(DEV), torch.tensor([700.0]), txt.unsqueeze(0).to(DEV),
                        pooled.unsqueeze(0).to(DEV))
    ref = osd.forward(sd, cfg.oracle_dict(), bf(lat), 700.0, bf(txt), bf(pooled))
    assert_close(out[0].cpu(), ref, 0.999, 2e-2, "sd35-medium 24 blocks")


def test_sd35_medium_1024_cfg_pair_full_step_matches_oracle():
    """The SD3.5-Medium 1024^2 CFG pair at full size (24 joint blocks, 13 dual; 2 x
    (4096 image + 333 text) joint tokens, packed) against the oracle run in fp32 on
    the GPU (torch's fp32 memory-efficient SDPA for its attention): each
    prediction within cos >= 0.999 and relative L2 <= 2e-2."""
    from oracle import common as oc
    sd35 = _sd()
    cfg = sd35.SD35_MEDIUM
    sd = sd35.random_state_dict(cfg, seed=4, device=DEV)
    model = sd35.SD35Transformer(cfg, sd, DEV)
    (lat, txt_c, pool_c), (_, txt_u, pool_u) = _inputs(30, 1024), _inputs(33, 1024)
    reqs = [(txt_u, pool_u), (txt_c, pool_c)]
    outs, meta = model.forward_packed([lat.to(DEV)] * 2, [900.0] * 2, [t.to(DEV) for t, _ in reqs],
                                      [p.to(DEV) for _, p in reqs])
    assert meta["cu_seqlens_joint"] == [0, 4429, 8858]
    outs = [o.cpu() for o in outs]
    del model
    torch.cuda.empty_cache()
    with torch.no_grad():
        for out, (txt, pooled), label in zip(outs, reqs, ("uncond", "cond")):
            ref = osd.forward(sd, cfg.oracle_dict(), bf(lat).to(DEV), 900.0, bf(txt).to(DEV), bf(pooled).to(DEV),
                              attn=oc.sdpa_fast)
            c, r = assert_close(out, ref.cpu(), 0.999, 2e-2, f"sd35-medium 1024 step ({label})")
            print(f"{label}: cos {c:.6f} relL2 {r:.3e}")


def test_sd35_config3_packed_cfg_batch_bitwise():
    """2 x 1024^2 + 4 x 512^2 requests, each as an (uncond, cond) CFG pair -> 12 packed
    segments; every segment equals its solo forward bitwise."""
    sd35 = _sd()
    cfg = sd35.SD35_MEDIUM
    model = sd35.SD35Transformer.random(cfg, seed=2, device=DEV)
    res = [1024, 1024, 512, 512, 512, 512]
    lats, ts, txts, pools = [], [], [], []
    for r, size in enumerate(res):
        lat, txt_c, pool_c = _inputs(20 + 3 * r, size)
        txt_u, pool_u = torch.zeros_like(txt_c), torch.zeros_like(pool_c)
        t = float(100 * (r + 1))
        for txt, pool in ((txt_u, pool_u), (txt_c, pool_c)):  # sd35.py:919-930 order
            lats.append(lat.to(DEV))
            ts.append(t)
            txts.append(txt.to(DEV))
            pools.append(pool.to(DEV))
    outs, meta = sd35.forward_packed_sd35(torch, model, [l.unsqueeze(0) for l in lats], ts,
                                          [t.unsqueeze(0) for t in txts], pools)
    from ditserve_amd.packing import build_cu_seqlens
    counts = [(s // 16) ** 2 for s in res for _ in range(2)]
    assert meta["cu_seqlens_img"] == build_cu_seqlens(counts)
    assert meta["cu_seqlens_joint"] == [a + 333 * i for i, a in enumerate(build_cu_seqlens(counts))]
    g = GOLD["sd35_packed"]  # the same request set without CFG duplication
    from ditserve_amd.packing import joint_layout
    lay = joint_layout(g["img_counts"], g["txt_counts"])
    assert lay["cu_img"] == g["cu_img"] and lay["cu_joint"] == g["cu_joint"]
    for i in (0, 1, 5, 11):
        solo, _ = sd35.forward_packed_sd35(torch, model, [lats[i].unsqueeze(0)], [ts[i]], [txts[i].unsqueeze(0)],
                                           [pools[i]])
        assert torch.isfinite(solo[0]).all()
        assert torch.equal(outs[i], solo[0]), f"segment {i} differs"


def test_sd35_config3_packed_cfg_batch_matches_oracle():
    """The packed 2 x 1024^2 + 4 x 512^2 CFG batch (12 joint segments, 24 blocks) at
    full size: every segment's prediction against the oracle run in fp32 on the GPU,
    cos >= 0.999 and relative L2 <= 2e-2."""
    from oracle import common as oc
    sd35 = _sd()
    cfg = sd35.SD35_MEDIUM
    sd = sd35.random_state_dict(cfg, seed=5, device=DEV)
    model = sd35.SD35Transformer(cfg, sd, DEV)
    res = [1024, 1024, 512, 512, 512, 512]
    segs = []
    for r, size in enumerate(res):
        lat, txt_c, pool_c = _inputs(40 + 3 * r, size)
        txt_u, pool_u = torch.zeros_like(txt_c), torch.zeros_like(pool_c)
        for txt, pool in ((txt_u, pool_u), (txt_c, pool_c)):
            segs.append((lat, float(75 * (r + 1)), txt, pool))
    outs, meta = model.forward_packed([x[0].to(DEV) for x in segs], [x[1] for x in segs],
                                      [x[2].to(DEV) for x in segs], [x[3].to(DEV) for x in segs])
    assert len(meta["cu_seqlens_joint"]) == 13
    outs = [o.cpu() for o in outs]
    del model
    torch.cuda.empty_cache()
    with torch.no_grad():
        for i, ((lat, t, txt, pool), out) in enumerate(zip(segs, outs)):
            ref = osd.forward(sd, cfg.oracle_dict(), bf(lat).to(DEV), t, bf(txt).to(DEV), bf(pool).to(DEV),
                              attn=oc.sdpa_fast)
            c, r = assert_close(out, ref.cpu(), 0.999, 2e-2, f"segment {i} ({res[i // 2]}^2, t={t})")
            print(f"segment {i} ({res[i // 2]}^2): cos {c:.6f} relL2 {r:.3e}")


REFERENCE_BATCH = {"results", "batch_size", "quantum", "model_ms", "attention", "bubble_free", "sequence_packing",
                   "packing", "step_meta", "memory_after"}
REFERENCE_META = {"sequence_packed", "attention_backend", "attention_provider", "packed_segments", "cu_seqlens_img",
                  "cu_seqlens_txt", "packed_image_tokens", "padded_image_tokens", "padding_saved_tokens"}


def _state(seed, res, steps, guidance):
    from ditserve_amd.solver import FlowMatchEulerScheduler
    lat, txt, pooled = _inputs(seed, res)
    sched = FlowMatchEulerScheduler(shift=3.0)
    sched.set_timesteps(steps)
    emb = dict(prompt_embeds=txt.unsqueeze(0).to(DEV), pooled_prompt_embeds=pooled.unsqueeze(0).to(DEV),
               negative_prompt_embeds=torch.zeros(1, 333, 4096, device=DEV),
               negative_pooled_prompt_embeds=torch.zeros(1, 2048, device=DEV))
    return dict(latents=lat.unsqueeze(0).to(DEV), timesteps=sched.timesteps, step=0,
                spec=dict(height=res, width=res, guidance_scale=guidance, steps=steps), embeds=emb, scheduler=sched)


def test_sd35_advance_batch_result_and_packing_invariance():
    """workers/ditserve/models/sd35.py:1025-1164: the batched advance of a mixed batch
    (two resolutions, one state without CFG) packs every segment, reports the
    reference's fields, and leaves each state where its solo advance leaves it."""
    sd35 = _sd()
    cfg = sd35.SD35Config(layers=3, dual_layers=(0,))
    model = sd35.SD35Transformer.random(cfg, seed=4, device=DEV)
    specs = [(60, 256, 2, 5.0), (61, 128, 2, 1.0)]
    states = [_state(*s) for s in specs]
    res = sd35.advance_batch(model, states, ["a", "b"], steps=1)
    assert set(res) == REFERENCE_BATCH and res["sequence_packing"] is True
    assert REFERENCE_META <= set(res["step_meta"]) and res["step_meta"]["packed_segments"] == 3
    assert res["packing"]["image_token_counts"] == [256, 64] and res["packing"]["heterogeneous_resolutions"]
    assert [r["progress"]["step"] for r in res["results"]] == [1, 1] and all(r["paused"] for r in res["results"])
    for s, st in zip(specs, states):
        solo = _state(*s)
        sd35.advance_batch(model, [solo], ["x"], steps=1)
        assert torch.equal(solo["latents"], st["latents"])
    res = sd35.advance_batch(model, states, ["a", "b"], steps=3)
    assert all(r["progress"]["done"] and not r["paused"] for r in res["results"])
    # homogeneous batch: the reference's dense form is reported (same packed kernels run)
    homo = [_state(70, 128, 1, 5.0), _state(71, 128, 1, 5.0)]
    res = sd35.advance_batch(model, homo, ["c", "d"])
    assert res["sequence_packing"] is False and res["step_meta"]["batch_size"] == 2
    forced = [_state(70, 128, 1, 5.0), _state(71, 128, 1, 5.0)]
    res2 = sd35.advance_batch(model, forced, ["c", "d"], sequence_packing=True)
    assert res2["sequence_packing"] is True
    for a, b in zip(homo, forced):
        assert torch.equal(a["latents"], b["latents"])
    with pytest.raises(ValueError):
        sd35.advance_batch(model, homo, ["c", "d"])  # both finished

"""The Wan engine (ditserve_amd.engine.DitkWanEngine) driven the way the
reference's block executor drives its engine: begin_packet per branch, every
forward_block, prediction, CFG combine, scheduler step
(workers/ditserve/models/wan/block.py:193-235,450-485).  Checked against the CPU
oracle; the whole-step ``forward`` and the interleaved side-stream mode
(block.py:237-300, its generic per-block path) against the sequential blocks,
bitwise."""
import types

import numpy as np
import pytest
import torch

from oracle import solver as osv
from oracle import wan as ow
from tests.helpers import assert_close, bf, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def tiny():
    from ditserve_amd.wan import WanConfig, WanTransformer, random_state_dict
    cfg = WanConfig(dim=256, heads=2, ffn=512, layers=3, text_dim=64)
    sd = random_state_dict(cfg, seed=11)
    return cfg, sd, WanTransformer(cfg, sd, DEV)


def _state(steps=8):
    from ditserve_amd.solver import UniPCFlowScheduler
    sched = UniPCFlowScheduler(flow_shift=3.0)
    sched.set_timesteps(steps)
    lat = bf(randn((1, 16, 3, 8, 12), 40))
    text = bf(randn((1, 20, 64), 41))
    text[:, 12:] = 0
    return types.SimpleNamespace(latents=lat.to(DEV), prompt_embeds=text.to(DEV),
                                 negative_prompt_embeds=torch.zeros(1, 20, 64, device=DEV), scheduler=sched,
                                 step_index=0, spec=dict(steps=steps, guidance_scale=5.0))


def _branch(engine, state, branch):
    packet = engine.begin_packet(state, branch)
    for i in range(engine.model.cfg.layers):
        packet["hidden"] = engine.forward_block(packet, i)
    return engine.prediction(packet)


def test_reference_call_order_matches_oracle(tiny):
    from ditserve_amd.engine import DitkWanEngine
    cfg, sd, model = tiny
    eng = DitkWanEngine(model)
    st = _state()
    eng.activate(st)
    lat0 = st.latents.clone()
    t = float(st.scheduler.timesteps[st.step_index])
    cond = _branch(eng, st, "cond")      # _finish_branch: conditional kept, branch -> uncond
    uncond = _branch(eng, st, "uncond")
    assert cond.shape == st.latents.shape
    pred = uncond + 5.0 * (cond - uncond)
    st.latents = st.scheduler.step(pred, st.scheduler.timesteps[st.step_index], st.latents)[0]
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    lat = lat0[0].cpu()
    rc = ow.forward(sd, ocfg, lat, t, st.prompt_embeds[0].cpu())
    ru = ow.forward(sd, ocfg, lat, t, st.negative_prompt_embeds[0].cpu())
    assert_close(cond[0].cpu(), rc, 0.999, 2e-2, "cond branch")
    assert_close(uncond[0].cpu(), ru, 0.999, 2e-2, "uncond branch")
    sigmas, _ = osv.unipc_flow_sigmas(8, 3.0)
    ref = osv.UniPCFlowOracle(sigmas).step(osv.cfg(rc.double().numpy(), ru.double().numpy(), 5.0),
                                           lat.double().numpy())
    x0 = lat.double()
    # branch errors (<= 2e-2 each, checked above) reach v = u + g (c - u) with weights g, g - 1
    c64, u64 = rc.double().numpy(), ru.double().numpy()
    tol = 2e-2 * (5.0 * np.linalg.norm(c64) + 4.0 * np.linalg.norm(u64)) / np.linalg.norm(osv.cfg(c64, u64, 5.0))
    assert_close(st.latents[0].cpu().double() - x0, torch.from_numpy(np.asarray(ref)) - x0, 0.999, tol,
                 "engine step delta")


def test_forward_equals_blockwise(tiny):
    from ditserve_amd.engine import DitkWanEngine
    _, _, model = tiny
    eng = DitkWanEngine(model)
    st = _state()
    assert torch.equal(eng.forward(st, "cond"), _branch(eng, st, "cond"))


def test_interleaved_side_stream_matches_sequential(tiny):
    """The reference's interleaved mode with an engine model that exposes no
    diffusers sublayers: block i of cond on the main stream, of uncond on a side
    stream, packets recorded on the side stream, one wait per quantum."""
    from ditserve_amd.engine import DitkWanEngine
    _, _, model = tiny
    eng = DitkWanEngine(model)
    st = _state()
    seq = (_branch(eng, st, "cond"), _branch(eng, st, "uncond"))
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    for _ in range(2):
        pc, pu = eng.begin_packet(st, "cond"), eng.begin_packet(st, "uncond")
        side.wait_stream(main)
        for v in pu.values():
            for t in (v if isinstance(v, (tuple, list)) else (v,)):
                if hasattr(t, "record_stream"):
                    t.record_stream(side)
        for i in range(model.cfg.layers):
            pc["hidden"] = eng.forward_block(pc, i)
            with torch.cuda.stream(side):
                pu["hidden"] = eng.forward_block(pu, i)
        main.wait_stream(side)
        out = (eng.prediction(pc), eng.prediction(pu))
        torch.cuda.synchronize()
        assert torch.equal(out[0], seq[0]) and torch.equal(out[1], seq[1])


def test_engine_surface(tiny):
    from ditserve_amd.engine import DitkWanEngine
    _, _, model = tiny
    eng = DitkWanEngine(model)
    info = eng.info()
    assert {"name", "revision", "attention", "sp_ranks", "pipeline", "transformer"} <= set(info)
    assert info["revision"] == eng.revision
    st = _state()
    with pytest.raises(ValueError):
        eng.activate(st, types.SimpleNamespace(ranks=(0, 1), degree=2, cfg=1))
    with pytest.raises(ValueError):
        eng.attach_groups([(0, 1)][0])
    with pytest.raises(ValueError):
        eng.begin_packet(st, "neither")
    bad = _state()
    bad.latents = bad.latents[:, :, :, :7]
    with pytest.raises(ValueError):
        eng.activate(bad)
    eng.close()
    with pytest.raises(RuntimeError):
        eng.activate(st)


def test_wan22_expand_timesteps():
    """Wan2.2 TI2V per-token timesteps (runtime.py:153-163) through the engine."""
    from ditserve_amd.engine import DitkWanEngine
    from ditserve_amd.wan import WanConfig, WanTransformer
    cfg = WanConfig(dim=256, heads=2, ffn=512, layers=1, in_ch=48, out_ch=48, text_dim=64)
    model = WanTransformer.random(cfg, seed=3, device=DEV)
    st = _state()
    st.latents = randn((1, 48, 3, 8, 12), 42).to(DEV)
    a = DitkWanEngine(model, expand_timesteps=True)
    b = DitkWanEngine(model)
    assert a._timestep(st).shape == (1, 3 * 4 * 6) and b._timestep(st).shape == (1,)
    assert torch.equal(a.forward(st, "cond"), b.forward(st, "cond"))

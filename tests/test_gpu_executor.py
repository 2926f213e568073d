"""Packed block executor on the GPU.

* Block quanta of any size, doorbell stops, and a mid-step export / import
  through the block-packet wire format reproduce the monolithic solver steps
  bitwise.
* The quantum rows, the manifest layout and the batched-advance result carry the
  reference's fields (workers/ditserve/models/wan/block.py:611-617,921-941;
  workers/ditserve/models/sd35.py:1148-1159).
* One packed executor step of a CFG pair matches the oracle: the CPU fp32 forward
  of each branch, the CFG combine and the float64 UniPC step (each branch's error
  bound carried through the guidance weights).
"""
import copy

import numpy as np
import pytest
import torch

from oracle import solver as osv
from oracle import wan as ow
from tests.helpers import assert_close, bf, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"

# the reference's row and manifest fields, written out here from block.py:611-617,921-941
REFERENCE_ROW = {"kind", "step_index", "branch", "start_block", "next_block", "next_branch", "blocks",
                 "step_completed", "ms", "doorbell_stop", "released_cache_on_stop", "block_cuda_ms",
                 "extra_state_bytes"}
REFERENCE_LAYOUT = {"committed_step", "branch", "next_block", "packet", "conditional", "folded"}
REFERENCE_PACKET_LAYOUT = {"shape", "rotary", "xdit", "engine"}
REFERENCE_MANIFEST = {"schema", "base", "layout", "packet_sha256", "strides"}
REFERENCE_BATCH = {"results", "batch_size", "quantum", "model_ms", "attention", "bubble_free", "sequence_packing",
                   "packing", "step_meta", "memory_after"}


def _requests(steps=6):
    from ditserve_amd.executor import Request
    reqs = []
    for i, (f, h, w) in enumerate(((3, 16, 24), (2, 10, 12))):
        reqs.append(Request(randn((16, f, h, w), 10 + i).to(DEV), randn((512, 4096), 20 + i).to(DEV),
                            torch.zeros(512, 4096, device=DEV), guidance_scale=5.0, steps=steps, request_id=f"r{i}"))
    return reqs


@pytest.fixture(scope="module")
def model():
    from ditserve_amd.wan import WanConfig, WanTransformer
    return WanTransformer.random(WanConfig(layers=4), seed=5, device=DEV)


def _clone(reqs):
    out = []
    for r in reqs:
        c = copy.copy(r)
        c.latents = r.latents.clone()
        c.scheduler = copy.deepcopy(r.scheduler)
        c.events = []
        out.append(c)
    return out


def test_row_field_sets_match_reference():
    from ditserve_amd.executor import BATCH_RESULT_FIELDS, PACKED_ROW_FIELDS, QUANTUM_ROW_FIELDS
    assert QUANTUM_ROW_FIELDS == REFERENCE_ROW
    assert BATCH_RESULT_FIELDS == REFERENCE_BATCH
    assert not (PACKED_ROW_FIELDS & REFERENCE_ROW)


def test_quanta_match_whole_steps(model):
    from ditserve_amd.executor import PACKED_ROW_FIELDS, PackedBlockExecutor
    base = _requests()
    a, b = _clone(base), _clone(base)
    ea, eb = PackedBlockExecutor(model), PackedBlockExecutor(model)
    ea.attach(a)
    eb.attach(b)
    for _ in range(2):
        rows = ea.step(observe=True)
        assert len(rows) == 2 and all(r["step_completed"] and r["blocks"] == 4 for r in rows)
        assert len(rows[0]["block_cuda_ms"]) == 4
    quanta = []
    while b[0].step_index < 2:
        quanta.append(eb.advance(3, observe=True))
    assert [q[0]["blocks"] for q in quanta] == [3, 1, 3, 1]
    assert [q[0]["next_block"] for q in quanta] == [3, 0, 3, 0]
    for q in quanta:
        for row, req in zip(q, b):
            assert set(row) == REFERENCE_ROW | PACKED_ROW_FIELDS
            assert row["request_id"] == req.request_id and row["branch"] == "cond+uncond" == row["next_branch"]
            assert row["doorbell_stop"] is False and row["released_cache_on_stop"] is False
    assert quanta[0][0]["packing"]["image_token_counts"] == [288, 288, 60, 60]
    assert quanta[0][0]["extra_state_bytes"] > 0 and quanta[1][0]["extra_state_bytes"] == 0
    assert [q[0]["step_index"] for q in quanta] == [0, 0, 1, 1]
    assert all(ev["ms"] > 0 for q in quanta for ev in q[0]["block_cuda_ms"])
    for x, y in zip(a, b):
        assert torch.equal(x.latents, y.latents)
        assert [e["completed_steps"] for e in y.events if e["kind"] == "step"] == [1, 2]


def test_doorbell_stop_and_resume_bitwise(model):
    from ditserve_amd.executor import PackedBlockExecutor
    base = _requests()
    a, b = _clone(base), _clone(base)
    ea = PackedBlockExecutor(model)
    ea.attach(a)
    ea.step()
    eb = PackedBlockExecutor(model, release_cache_on_stop=True)
    eb.attach(b)
    calls = []

    def bell():
        calls.append(1)
        return len(calls) == 2
    rows = eb.advance(4, doorbell=bell, check_every=1)
    assert rows[0]["doorbell_stop"] and rows[0]["next_block"] == 2 and rows[0]["blocks"] == 2
    assert rows[0]["released_cache_on_stop"] and not rows[0]["step_completed"]
    rows = eb.advance(4, doorbell=lambda: False, check_every=1)
    assert rows[0]["step_completed"] and not rows[0]["doorbell_stop"] and rows[0]["start_block"] == 2
    for x, y in zip(a, b):
        assert torch.equal(x.latents, y.latents)
    with pytest.raises(ValueError):
        eb.advance(2, doorbell=bell)  # a doorbell needs check_every


def test_mid_step_export_import_resumes_bitwise(model):
    from ditserve_amd.executor import PackedBlockExecutor
    base = _requests()
    a, b = _clone(base), _clone(base)
    ea = PackedBlockExecutor(model)
    ea.attach(a)
    for _ in range(3):
        ea.step()
    eb = PackedBlockExecutor(model)
    eb.attach(b)
    eb.step()
    eb.step()
    eb.advance(2)
    payload, stats = eb.export()
    man = payload["manifest"]
    assert set(man) == REFERENCE_MANIFEST
    assert REFERENCE_LAYOUT | REFERENCE_PACKET_LAYOUT <= set(man["layout"])
    assert man["layout"]["next_block"] == 2 and man["layout"]["packet"] and man["layout"]["committed_step"] == [2, 2]
    assert set(man["layout"]["xdit"]) == {"pad_amount", "local_rows", "valid_kv_len", "thw"}
    assert stats["packet_bytes"] > 0 and stats["transfer_bytes"] > stats["packet_bytes"]
    del eb
    ec = PackedBlockExecutor.import_state(payload, model)
    rows = ec.advance(8)
    assert rows[0]["start_block"] == 2 and rows[0]["step_completed"]
    for x, y in zip(a, ec.requests):
        assert torch.equal(x.latents, y.latents)
        assert x.step_index == y.step_index == 3
    # a second step after the import still agrees (solver history carried over)
    ea.step()
    ec.step()
    for x, y in zip(a, ec.requests):
        assert torch.equal(x.latents, y.latents)
    # tampering is rejected
    bad = {"manifest": copy.deepcopy(man), "tensors": dict(payload["tensors"])}
    bad["tensors"]["packet.hidden"] = payload["tensors"]["packet.hidden"].clone()
    bad["tensors"]["packet.hidden"].view(-1)[0] += 1
    with pytest.raises(ValueError):
        PackedBlockExecutor.import_state(bad, model)
    bad = {"manifest": copy.deepcopy(man), "tensors": dict(payload["tensors"])}
    bad["manifest"]["base"]["requests"][0]["guidance_scale"] = 7.0
    with pytest.raises(ValueError):
        PackedBlockExecutor.import_state(bad, model)
    bad = {"manifest": copy.deepcopy(man), "tensors": dict(payload["tensors"])}
    bad["manifest"]["layout"]["committed_step"] = [1, 2]
    with pytest.raises(ValueError):
        PackedBlockExecutor.import_state(bad, model)


def test_step_boundary_export_import(model):
    from ditserve_amd.executor import PackedBlockExecutor
    base = _requests()
    a, b = _clone(base), _clone(base)
    ea = PackedBlockExecutor(model)
    ea.attach(a)
    ea.step()
    ea.step()
    eb = PackedBlockExecutor(model)
    eb.attach(b)
    eb.step()
    payload, stats = eb.export()
    assert payload["manifest"]["layout"]["packet"] is False and stats["packet_bytes"] == 0
    ec = PackedBlockExecutor.import_state(payload, model)
    ec.step()
    for x, y in zip(a, ec.requests):
        assert torch.equal(x.latents, y.latents)


def test_advance_batch_result(model):
    from ditserve_amd.executor import PackedBlockExecutor
    base = _requests(steps=3)
    a, b = _clone(base), _clone(base)
    ea = PackedBlockExecutor(model)
    ea.attach(a)
    for _ in range(2):
        ea.step()
    eb = PackedBlockExecutor(model)
    eb.attach(b)
    res = eb.advance_batch(2, state_ids=["s0", "s1"])
    assert set(res) == REFERENCE_BATCH
    assert res["batch_size"] == 2 and res["quantum"] == "continuous_batch" and res["sequence_packing"]
    assert [r["state_id"] for r in res["results"]] == ["s0", "s1"]
    assert res["results"][0]["progress"] == dict(step=2, steps=3, done=False, next_action="advance")
    assert res["results"][0]["paused"] is True and res["model_ms"] > 0
    assert res["packing"]["cu_seqlens"] == [0, 288, 576, 636, 696]
    assert res["step_meta"]["cu_seqlens_img"] == [0, 288, 576, 636, 696]
    for x, y in zip(a, b):
        assert torch.equal(x.latents, y.latents)
    res = eb.advance_batch(5, state_ids=["s0", "s1"])
    assert all(r["progress"]["done"] and not r["paused"] for r in res["results"])


def test_packed_step_matches_oracle():
    """One executor step of a CFG pair on a tiny Wan configuration against the CPU
    oracle: each branch's fp32 forward, the CFG combine and the float64 UniPC step.
    The latent change x' - x is compared (the latent itself would hide errors)."""
    from ditserve_amd.executor import PackedBlockExecutor, Request
    from ditserve_amd.wan import WanConfig, WanTransformer, random_state_dict
    cfg = WanConfig(dim=256, heads=2, ffn=512, layers=2, text_dim=64)
    sd = random_state_dict(cfg, seed=7)
    model = WanTransformer(cfg, sd, DEV)
    lat = bf(randn((16, 3, 8, 12), 30))
    text = bf(randn((24, 64), 31))
    text[10:] = 0
    neg = torch.zeros(24, 64)
    req = Request(lat.to(DEV), text.to(DEV), neg.to(DEV), guidance_scale=5.0, steps=10, flow_shift=3.0)
    t = float(req.scheduler.timesteps[0])
    ex = PackedBlockExecutor(model)
    ex.attach([req])
    ex.step()
    got = req.latents.cpu().double()
    ocfg = dict(patch=cfg.patch, head_dim=cfg.head_dim, heads=cfg.heads, layers=cfg.layers, freq_dim=cfg.freq_dim,
                eps=cfg.eps, out_ch=cfg.out_ch)
    cond = ow.forward(sd, ocfg, lat, t, text).double().numpy()
    uncond = ow.forward(sd, ocfg, lat, t, neg).double().numpy()
    sigmas, _ = osv.unipc_flow_sigmas(10, 3.0)
    ref = osv.UniPCFlowOracle(sigmas).step(osv.cfg(cond, uncond, 5.0), lat.double().numpy())
    x0 = lat.double()
    # Each branch is held to relative L2 2e-2; the CFG combine v = u + g (c - u)
    # carries those errors into v with weights g and g - 1, so the step's change
    # is held to the propagated bound 2e-2 (g |c| + (g - 1) |u|) / |v|.
    v = osv.cfg(cond, uncond, 5.0)
    tol = 2e-2 * (5.0 * np.linalg.norm(cond) + 4.0 * np.linalg.norm(uncond)) / np.linalg.norm(v)
    assert_close(got - x0, torch.from_numpy(np.asarray(ref)) - x0, 0.999, tol, "packed step delta")
    assert_close(got, torch.from_numpy(np.asarray(ref)), 0.9999, 2e-3, "packed step latent")

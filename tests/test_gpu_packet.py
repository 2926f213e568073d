"""Block-packet wire format: a packet exported at a block boundary and rebuilt
from the manifest and CPU tensors alone resumes to results bitwise equal to an
uninterrupted run; tampered payloads are rejected."""
import json

import pytest
import torch

from tests.helpers import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(layers=4):
    from ditserve_amd.wan import WanConfig, WanTransformer
    cfg = WanConfig(layers=layers)
    model = WanTransformer.random(cfg, seed=3, device=DEV)
    lats = [randn((16, 3, 16, 24), 1).to(DEV), randn((16, 2, 10, 12), 2).to(DEV)]
    texts = [randn((512, 4096), 3).to(DEV), randn((512, 4096), 4).to(DEV)]
    return model, lats, [640.0, 55.0], texts


@pytest.mark.parametrize("cut", [0, 2, 4])
def test_export_import_resumes_bitwise(cut):
    from ditserve_amd.packet import export_packet, import_packet
    model, lats, ts, texts = _setup()
    ref = model.forward_packed(lats, ts, texts)
    pk = model.begin_packed_packet(lats, ts, texts)
    for i in range(cut):
        model.forward_block(pk, i)
    payload, stats = export_packet(pk)
    json.dumps(payload["manifest"])  # the manifest is plain JSON
    assert all(t.device.type == "cpu" and t.is_contiguous() for t in payload["tensors"].values())
    assert stats["packet_bytes"] > 0
    del pk
    pk2 = import_packet(payload, model)
    for i in range(cut, model.cfg.layers):
        model.forward_block(pk2, i)
    outs = model.prediction_packed(pk2)
    for a, b in zip(outs, ref):
        assert torch.equal(a, b)


def test_import_rejects_tampered_payloads():
    from ditserve_amd.packet import export_packet, import_packet
    model, lats, ts, texts = _setup(layers=1)
    pk = model.begin_packed_packet(lats, ts, texts)
    payload, _ = export_packet(pk)
    bad = dict(payload, tensors=dict(payload["tensors"]))
    t = bad["tensors"]["packet.hidden"].clone()
    t.view(torch.int16)[0, 0] ^= 1
    bad["tensors"]["packet.hidden"] = t
    with pytest.raises(ValueError, match="checksum"):
        import_packet(bad, model)
    with pytest.raises(ValueError, match="schema"):
        import_packet(dict(payload, manifest=dict(payload["manifest"], schema="other")), model)
    missing = dict(payload, tensors={k: v for k, v in payload["tensors"].items() if k != "packet.temb"})
    with pytest.raises(ValueError, match="tensor set"):
        import_packet(missing, model)
    other = dict(payload["manifest"], layout=dict(payload["manifest"]["layout"], engine={"revision": "x"}))
    with pytest.raises(ValueError, match="revision"):
        import_packet(dict(payload, manifest=other), model)

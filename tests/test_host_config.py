"""Host-side configuration mirrors: diffusers transformer configs map onto the
architectures the kernels are built for, and unsupported variants are refused."""
import pytest

from ditserve_amd.sd35 import SD35_MEDIUM, SD35Config
from ditserve_amd.wan import WAN21_T2V_1_3B, WAN22_TI2V_5B, WanConfig

# diffusers WanTransformer3DModel constructor arguments of the Wan2.1-T2V-1.3B and
# Wan2.2-TI2V-5B checkpoints
WAN21 = dict(patch_size=[1, 2, 2], num_attention_heads=12, attention_head_dim=128, in_channels=16, out_channels=16,
             text_dim=4096, freq_dim=256, ffn_dim=8960, num_layers=30, cross_attn_norm=True,
             qk_norm="rms_norm_across_heads", eps=1e-6, image_dim=None, added_kv_proj_dim=None, rope_max_seq_len=1024)
WAN22 = dict(WAN21, num_attention_heads=24, ffn_dim=14336, in_channels=48, out_channels=48)
# diffusers SD3Transformer2DModel constructor arguments of SD3.5-Medium
SD35M = dict(sample_size=128, patch_size=2, in_channels=16, num_layers=24, attention_head_dim=64,
             num_attention_heads=24, joint_attention_dim=4096, caption_projection_dim=1536,
             pooled_projection_dim=2048, out_channels=16, pos_embed_max_size=384,
             dual_attention_layers=tuple(range(13)), qk_norm="rms_norm")


def test_wan_configs_from_diffusers():
    assert WanConfig.from_diffusers(WAN21) == WAN21_T2V_1_3B
    assert WanConfig.from_diffusers(WAN22) == WAN22_TI2V_5B

    class Obj:
        pass
    o = Obj()
    o.__dict__.update(WAN21)
    assert WanConfig.from_diffusers(o) == WAN21_T2V_1_3B


@pytest.mark.parametrize("change", [dict(image_dim=1280), dict(added_kv_proj_dim=1536), dict(qk_norm="rms_norm"),
                                    dict(cross_attn_norm=False)])
def test_wan_config_refuses_other_variants(change):
    with pytest.raises(ValueError):
        WanConfig.from_diffusers(dict(WAN21, **change))


def test_sd35_config_from_diffusers():
    assert SD35Config.from_diffusers(SD35M) == SD35_MEDIUM
    with pytest.raises(ValueError):
        SD35Config.from_diffusers(dict(SD35M, qk_norm=None))


def test_slot_rope_cache_is_keyed_on_the_table_tensors(monkeypatch):
    """The fused_qk_norm_rope slot reuses its rotation tables only for the very table
    tensors it built them from, alive and unmodified.  A fresh table of the same shape
    (the reference builds new ones per packet, transformer_wan.py:326), even when the
    allocator hands it a freed table's storage, gets tables of its own."""
    import torch

    from ditserve_amd import wan

    built = []

    class FakeRope:
        def __init__(self, cos_tab, sin_tab, *a):
            self.cos = cos_tab
            built.append(self)
    monkeypatch.setattr(wan.ops, "Rope", FakeRope)
    monkeypatch.setattr(wan, "Segments", lambda cu, device: None)
    monkeypatch.setattr(wan, "_SLOT_ROPE", [])
    S, dh = 6, 8
    storage = torch.arange(S * dh, dtype=torch.float32)
    c1, s1 = storage.view(1, S, 1, dh), torch.zeros(1, S, 1, dh)
    r1 = wan._slot_rope(c1, s1, "cpu", 1, S, dh)
    assert wan._slot_rope(c1, s1, "cpu", 1, S, dh) is r1           # same live tables: cached
    del c1
    c2 = storage.view(1, S, 1, dh)                                  # same address, new tensor
    r2 = wan._slot_rope(c2, s1, "cpu", 1, S, dh)
    assert r2 is not r1 and len(built) == 2
    c2.mul_(2.0)                                                    # modified in place: rebuilt
    r3 = wan._slot_rope(c2, s1, "cpu", 1, S, dh)
    assert r3 is not r2 and torch.equal(r3.cos, c2.reshape(S, dh)[:, 0::2])
    assert wan._slot_rope(c2, s1, "cpu", 2, S, dh) is not r3        # other batch size: rebuilt


def test_slot_norm_arguments():
    """The slot's norm_q / norm_k may be RMSNorm modules (their weight and eps, the
    input dtype's epsilon when torch.nn.RMSNorm's eps is None, unit weights without
    an elementwise affine) or bare weight tensors (eps 1e-6)."""
    import torch

    from ditserve_amd import wan

    q = torch.zeros(2, 3, 8, dtype=torch.bfloat16)
    m = torch.nn.RMSNorm(8, eps=1e-5)
    with torch.no_grad():
        m.weight.copy_(torch.arange(8.0))
    w, eps = wan._slot_norm(m, 8, q)
    assert torch.equal(w, torch.arange(8.0)) and eps == 1e-5
    w, eps = wan._slot_norm(torch.nn.RMSNorm(8), 8, q)
    assert eps == torch.finfo(torch.bfloat16).eps
    w, eps = wan._slot_norm(torch.nn.RMSNorm(8, eps=1e-6, elementwise_affine=False), 8, q)
    assert torch.equal(w, torch.ones(8)) and eps == 1e-6
    w, eps = wan._slot_norm(torch.full((8,), 2.0, dtype=torch.bfloat16), 8, q)
    assert w.dtype == torch.float32 and torch.equal(w, torch.full((8,), 2.0)) and eps == 1e-6


def test_view_extent_and_overlap():
    """linear_pair's aliasing check: byte ranges of strided views."""
    import torch

    from ditserve_amd import ops
    base = torch.zeros(10, 8, dtype=torch.bfloat16)
    a, b = base[:4], base[4:]
    assert ops._extent(a) == (a.data_ptr(), a.data_ptr() + 4 * 8 * 2)
    assert not ops._overlap(a, b) and ops._overlap(base, b) and ops._overlap(a, base[3:5])
    cols = base[:, 2:4]                                  # strided column slice: rows 0..9
    assert ops._extent(cols) == (cols.data_ptr(), cols.data_ptr() + (9 * 8 + 2) * 2)
    assert ops._overlap(cols, base[9:]) and not ops._overlap(base[:, :2][:1], base[:, 2:4][:1])
    assert ops._extent(base[:0]) == (0, 0) and not ops._overlap(base[:0], base)


def test_model_inputs_refused_before_any_launch():
    """Wrong latent channels / grids, text widths or SD3 patch counts raise
    ValueError before the first kernel (checked here on the CPU, no library call)."""
    import torch

    from ditserve_amd import sd35, wan
    w = wan.WanTransformer.__new__(wan.WanTransformer)
    w.cfg, w.device = wan.WAN21_T2V_1_3B, "cpu"
    lat = torch.zeros(16, 3, 8, 8)
    for lats, texts in (([torch.zeros(4, 3, 8, 8)], [torch.zeros(512, 4096)]),   # channels
                        ([torch.zeros(16, 3, 7, 8)], [torch.zeros(512, 4096)]),   # H not a patch multiple
                        ([lat], [torch.zeros(512, 2048)]),                        # text width
                        ([lat, lat], [torch.zeros(512, 4096)])):                  # list lengths
        with pytest.raises(ValueError):
            w.begin_packed_packet(lats, [500.0] * len(lats), texts)
    s = sd35.SD35Transformer.__new__(sd35.SD35Transformer)
    s.cfg, s.device = sd35.SD35_MEDIUM, "cpu"
    for lat, txt in (((16, 800, 64), (10, 4096)), ((16, 64, 64), (10, 2048)), ((4, 64, 64), (10, 4096))):
        with pytest.raises(ValueError):
            s.forward_packed([torch.zeros(lat)], [1.0], [torch.zeros(txt)], [torch.zeros(2048)])


def test_attention_plugin_dataclasses_match_reference():
    """The plugin's call objects carry the reference's fields
    (workers/xfuser/core/attention/spec.py:63-102), so a caller that builds them
    by keyword builds ours the same way."""
    import dataclasses

    from ditserve_amd import attention

    assert [f.name for f in dataclasses.fields(attention.VarlenPacking)] == [
        "indices_k", "cu_seqlens_k", "max_seqlen_k"]
    assert [f.name for f in dataclasses.fields(attention.AttnCall)] == [
        "dropout_p", "is_causal", "varlen", "ulysses_world_size", "ring_world_size", "attention_kwargs"]
    call = attention.AttnCall(ulysses_world_size=2, ring_world_size=2, attention_kwargs={"attn_mask": 1})
    assert call.attention_kwargs["attn_mask"] == 1
    assert attention.VarlenPacking.from_kwargs(None) is None
    assert attention.VarlenPacking.from_kwargs({"cu_seqlens_k": 1}) is None
    p = attention.VarlenPacking.from_kwargs({"indices_k": "i", "cu_seqlens_k": "c", "max_seqlen_k": 7})
    assert (p.indices_k, p.cu_seqlens_k, p.max_seqlen_k) == ("i", "c", 7)

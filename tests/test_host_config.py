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

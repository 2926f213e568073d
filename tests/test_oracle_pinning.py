"""Pin the oracle against things it does not restate: library routines (float64),
closed forms, invariants and special cases.  Each check is chosen so that a
plausible mistake (dropped term, wrong sign, swapped index/operand) fails it;
the planted-mistake tests at the end demonstrate that on the CPU."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import common as oc
from oracle import sd35 as osd
from oracle import wan as ow

D64 = torch.float64


def g(seed):
    return torch.Generator().manual_seed(seed)


# ----------------------------------------------------------------- primitives
def test_layer_norm_matches_library():
    x = torch.randn(7, 96, generator=g(0), dtype=D64) * 3 + 1
    w, b = torch.randn(96, generator=g(1), dtype=D64), torch.randn(96, generator=g(2), dtype=D64)
    assert torch.allclose(oc.layer_norm(x, 1e-6), F.layer_norm(x, (96,), eps=1e-6), atol=1e-12)
    assert torch.allclose(oc.layer_norm(x, 1e-6, w, b), F.layer_norm(x, (96,), w, b, eps=1e-6), atol=1e-12)


def test_rms_norm_matches_library():
    x = torch.randn(5, 128, generator=g(3), dtype=D64)
    w = torch.randn(128, generator=g(4), dtype=D64)
    assert torch.allclose(oc.rms_norm(x, w, 1e-6), F.rms_norm(x, (128,), w, eps=1e-6), atol=1e-12)


def test_gelu_tanh_and_silu_match_library():
    x = torch.linspace(-8, 8, 1001, dtype=D64)
    assert torch.allclose(oc.gelu_tanh(x), F.gelu(x, approximate="tanh"), atol=1e-12)
    assert torch.allclose(oc.silu(x), F.silu(x), atol=1e-12)


def test_timestep_embedding_closed_form():
    t = torch.tensor([0.0, 1.0, 999.0])
    e = oc.timestep_embedding(t, 256)
    assert torch.equal(e[0, :128], torch.ones(128)) and torch.equal(e[0, 128:], torch.zeros(128))
    for k in (0, 5, 127):
        f = math.exp(-math.log(10000.0) * k / 128)
        assert abs(float(e[2, k]) - math.cos(999.0 * f)) < 2e-4      # cos half first
        assert abs(float(e[2, 128 + k]) - math.sin(999.0 * f)) < 2e-4


def test_sdpa_matches_library_and_brute_force():
    q = torch.randn(2, 5, 16, generator=g(5), dtype=D64)
    k = torch.randn(2, 9, 16, generator=g(6), dtype=D64)
    v = torch.randn(2, 9, 8, generator=g(7), dtype=D64)
    ref = F.scaled_dot_product_attention(q, k, v)
    assert torch.allclose(oc.sdpa(q, k, v, chunk=2), ref, atol=1e-12)
    assert torch.allclose(oc.sdpa_fast(q, k, v), ref, atol=1e-12)
    out, lse = oc.sdpa_lse(q, k, v)
    # brute force for one query
    s = [sum(float(q[1, 3, d]) * float(k[1, j, d]) for d in range(16)) / 4.0 for j in range(9)]
    mx = max(s)
    den = sum(math.exp(x - mx) for x in s)
    o0 = sum(math.exp(s[j] - mx) / den * float(v[1, j, 0]) for j in range(9))
    assert abs(o0 - float(out[1, 3, 0])) < 1e-12
    assert abs(mx + math.log(den) - float(lse[1, 3])) < 1e-12


def test_varlen_attention_is_block_diagonal():
    cu = [0, 7, 19]  # the reference's joint dispatch (test_domain_block_executor.py:915)
    q = torch.randn(19, 2, 4, generator=g(8), dtype=D64)
    k = torch.randn(19, 2, 4, generator=g(9), dtype=D64)
    v = torch.randn(19, 2, 4, generator=g(10), dtype=D64)
    out = oc.varlen_attention(q, k, v, cu, cu)
    k2, v2 = k.clone(), v.clone()
    k2[7:] += 5.0
    v2[7:] -= 3.0
    out2 = oc.varlen_attention(q, k2, v2, cu, cu)
    assert torch.equal(out[:7], out2[:7])          # segment 0 blind to segment 1
    ref1 = F.scaled_dot_product_attention(q[7:].transpose(0, 1), k[7:].transpose(0, 1), v[7:].transpose(0, 1))
    assert torch.allclose(out[7:], ref1.transpose(0, 1), atol=1e-12)


# ----------------------------------------------------------------- RoPE
def test_rope_table_closed_form_and_axis_split():
    assert ow.rope_axis_split(128) == (44, 42, 42)
    cos, sin = ow.rope_table(128, 1024)
    for pair, pos in ((0, 5), (10, 700), (21, 33), (22, 9), (42, 1023), (43, 17), (63, 511)):
        f, h, w = pos, pos, pos
        ang = ow.rope_pair_angle(pair, f, h, w)
        assert abs(float(cos[pos, 2 * pair]) - math.cos(ang)) < 1e-6
        assert abs(float(sin[pos, 2 * pair + 1]) - math.sin(ang)) < 1e-6
        assert float(cos[pos, 2 * pair]) == float(cos[pos, 2 * pair + 1])  # repeat-interleaved


def test_rope_grid_positions():
    grid = (3, 4, 5)
    cos, _ = ow.rope_freqs(grid)
    table, _ = ow.rope_table(128, 1024)
    tok = (2 * 4 + 1) * 5 + 3  # f=2, h=1, w=3
    assert torch.equal(cos[tok, :44], table[2, :44])
    assert torch.equal(cos[tok, 44:86], table[1, 44:86])
    assert torch.equal(cos[tok, 86:], table[3, 86:])


def test_apply_rotary_is_complex_multiplication():
    """out = x * e^{i theta} on (x[2i] + i x[2i+1]) pairs — pins the sign convention
    of transformer_wan.py:183-186, which norm / relative-position invariants alone do not."""
    grid = (2, 3, 4)
    cos, sin = ow.rope_freqs(grid)
    x = torch.randn(24, 3, 128, generator=g(11))
    out = ow.apply_rotary(x, cos, sin)
    xc = torch.view_as_complex(x.reshape(24, 3, 64, 2).contiguous())
    rot = torch.polar(torch.ones(24, 64), torch.atan2(sin[:, 1::2], cos[:, 0::2]))
    ref = torch.view_as_real(xc * rot[:, None, :]).reshape(24, 3, 128)
    assert torch.allclose(out, ref, atol=1e-5)
    # identity at position 0 and pair-norm preservation
    assert torch.allclose(out[0], x[0], atol=1e-6)
    assert torch.allclose(out.reshape(24, 3, 64, 2).norm(dim=-1), x.reshape(24, 3, 64, 2).norm(dim=-1), atol=1e-5)


# ----------------------------------------------------------------- Wan pieces
def _tiny_wan(seed=0, layers=1):
    from ditserve_amd.wan import WanConfig, random_state_dict
    cfg = WanConfig(dim=256, heads=2, ffn=512, layers=layers, text_dim=64)
    return cfg, {k: v.double() for k, v in random_state_dict(cfg, seed).items()}


def test_patch_embed_matches_conv3d():
    cfg, p = _tiny_wan()
    lat = torch.randn(16, 3, 8, 10, generator=g(12), dtype=D64)
    ref = F.conv3d(lat[None], p["patch_embedding.weight"], p["patch_embedding.bias"], stride=(1, 2, 2))
    assert torch.allclose(ow.patch_embed(p, lat), ref.flatten(2)[0].t(), atol=1e-10)


def test_prediction_unpatchify_index_map():
    cfg, p = _tiny_wan()
    grid = (2, 3, 4)
    hidden = torch.randn(24, 256, generator=g(13), dtype=D64)
    temb = torch.randn(256, generator=g(14), dtype=D64)
    out = ow.prediction(p, hidden, temb, grid, 16)
    shift, scale = (p["scale_shift_table"].reshape(2, -1) + temb).unbind(0)
    y = F.linear(F.layer_norm(hidden, (256,), eps=1e-6) * (1 + scale) + shift, p["proj_out.weight"], p["proj_out.bias"])
    f, hh, ww, c = 1, 2, 3, 7  # output voxel (c, f, 2*? ...) check one element explicitly
    tok = (f * 3 + hh // 2) * 4 + ww // 2
    feat = ((0 * 2 + hh % 2) * 2 + ww % 2) * 16 + c
    assert abs(float(out[c, f, hh, ww]) - float(y[tok, feat])) < 1e-10


def test_condition_embedder_matches_module_composition():
    cfg, p = _tiny_wan()
    t = torch.tensor([500.0])
    text = torch.randn(6, 64, generator=g(15), dtype=D64)
    temb, proj, enc = ow.condition_embedder(p, t, text)
    pre = "condition_embedder"
    te = torch.nn.Sequential(torch.nn.Linear(256, 256), torch.nn.SiLU(), torch.nn.Linear(256, 256)).double()
    te[0].weight.data, te[0].bias.data = p[f"{pre}.time_embedder.linear_1.weight"], p[f"{pre}.time_embedder.linear_1.bias"]
    te[2].weight.data, te[2].bias.data = p[f"{pre}.time_embedder.linear_2.weight"], p[f"{pre}.time_embedder.linear_2.bias"]
    with torch.no_grad():
        ref = te(oc.timestep_embedding(t, 256).double())
    assert torch.allclose(temb, ref, atol=1e-10)
    assert proj.shape == (1, 6, 256) and enc.shape == (6, 256)
    # projected = time_proj(SiLU(temb)) unflattened as 6 chunks of D (transformer_wan.py:334-338;
    # block.py:276-280 then reads chunk j as the j-th modulation vector)
    tp = torch.nn.Sequential(torch.nn.SiLU(), torch.nn.Linear(256, 6 * 256)).double()
    tp[1].weight.data, tp[1].bias.data = p[f"{pre}.time_proj.weight"], p[f"{pre}.time_proj.bias"]
    with torch.no_grad():
        flat = tp(ref)[0]
    for j in range(6):
        assert torch.allclose(proj[0, j], flat[j * 256:(j + 1) * 256], atol=1e-10)
    # closed form: zero time_proj weight leaves the bias, chunk j = bias[j*D:(j+1)*D]
    q = dict(p)
    q[f"{pre}.time_proj.weight"] = torch.zeros_like(p[f"{pre}.time_proj.weight"])
    q[f"{pre}.time_proj.bias"] = torch.arange(6 * 256, dtype=D64)
    _, proj0, _ = ow.condition_embedder(q, t, text)
    assert torch.equal(proj0[0], torch.arange(6 * 256, dtype=D64).reshape(6, 256))
    tx = torch.nn.Sequential(torch.nn.Linear(64, 256), torch.nn.GELU(approximate="tanh"), torch.nn.Linear(256, 256)).double()
    tx[0].weight.data, tx[0].bias.data = p[f"{pre}.text_embedder.linear_1.weight"], p[f"{pre}.text_embedder.linear_1.bias"]
    tx[2].weight.data, tx[2].bias.data = p[f"{pre}.text_embedder.linear_2.weight"], p[f"{pre}.text_embedder.linear_2.bias"]
    with torch.no_grad():
        assert torch.allclose(enc, tx(text), atol=1e-10)


def test_wan_block_residual_structure():
    """Zero gates reduce the block to h + cross-attention (block.py:285,290,293)."""
    cfg, p = _tiny_wan()
    h = torch.randn(12, 256, generator=g(16), dtype=D64)
    enc = torch.randn(5, 256, generator=g(17), dtype=D64)
    cos, sin = ow.rope_freqs((1, 3, 4))
    sst = p["blocks.0.scale_shift_table"].reshape(6, -1)
    proj = torch.randn(6, 256, generator=g(18), dtype=D64)
    proj[2] = -sst[2]  # gate_msa = 0
    proj[5] = -sst[5]  # c_gate = 0
    out = ow.block_forward(p, 0, h, enc, proj, cos, sin, 2)
    n = F.layer_norm(h, (256,), p["blocks.0.norm2.weight"], p["blocks.0.norm2.bias"], eps=1e-6)
    assert torch.allclose(out, h + ow.cross_attention(p, "blocks.0.attn2", n, enc, 2), atol=1e-10)
    # the FFN branch is linear in c_gate
    proj2 = proj.clone()
    proj2[5] = -sst[5] + 1.0
    proj3 = proj.clone()
    proj3[5] = -sst[5] + 2.0
    o2, o3 = ow.block_forward(p, 0, h, enc, proj2, cos, sin, 2), ow.block_forward(p, 0, h, enc, proj3, cos, sin, 2)
    assert torch.allclose(o3 - out, 2 * (o2 - out), atol=1e-9)


def test_wan_qk_norm_is_across_heads():
    """rms_norm_across_heads: one RMS over all D, not per head (transformer_wan.py:165-166)."""
    q = torch.randn(3, 256, generator=g(19), dtype=D64)
    q[:, :128] *= 10
    w = torch.ones(256, dtype=D64)
    out, _ = ow.qk_norm_rope(q, q, w, w, None, None, 2)
    assert torch.allclose(out.flatten(1).pow(2).mean(-1), torch.ones(3, dtype=D64), atol=1e-5)
    assert not torch.allclose(out[:, 1].pow(2).mean(-1), torch.ones(3, dtype=D64), atol=1e-2)


# ----------------------------------------------------------------- SD3.5 pieces
def test_sd35_pos_embed_closed_form_and_crop():
    table = osd.pos_embed_table(64, max_size=384, base_size=64)
    r, c = 200, 31
    row = table[r * 384 + c]
    for k in (0, 7, 15):
        w = 1.0 / 10000 ** (k / 16.0)
        assert abs(float(row[k]) - math.sin((c * 64 / 384) * w)) < 1e-6          # column, sin
        assert abs(float(row[16 + k]) - math.cos((c * 64 / 384) * w)) < 1e-6     # column, cos
        assert abs(float(row[32 + k]) - math.sin((r * 64 / 384) * w)) < 1e-6     # row, sin
    crop = osd.cropped_pos_embed(table, 64, 64)
    assert torch.equal(crop[0], table[160 * 384 + 160])  # centre crop of a 1024^2 image
    from ditserve_amd.sd35 import SD35Config, pos_embed_crop
    prod = pos_embed_crop(SD35Config(dim=64), 64, 64, "cpu")
    assert torch.allclose(prod, crop, atol=1e-6)
    # a 192-wide table (SD3.5-Large's pos_embed_max_size): the crop of a 16 x 16 grid
    # starts at row = column = 88, coordinates i * 64 / 192
    t192 = osd.pos_embed_table(64, max_size=192, base_size=64)
    c192 = osd.cropped_pos_embed(t192, 16, 16)
    assert c192.shape == (256, 64)
    r, c = 88 + 3, 88 + 5
    w = 1.0 / 10000 ** (2 / 16.0)
    assert abs(float(c192[3 * 16 + 5, 2]) - math.sin((c * 64 / 192) * w)) < 1e-6
    assert abs(float(c192[3 * 16 + 5, 32 + 2]) - math.sin((r * 64 / 192) * w)) < 1e-6
    assert torch.allclose(pos_embed_crop(SD35Config(dim=64, pos_max=192), 16, 16, "cpu"), c192, atol=1e-6)
    # a non-square grid (40 patch rows x 72 patch columns, e.g. 640 x 1152 pixels): rows crop
    # from 172, columns from 156, tokens row-major; a transposed crop fails here
    cn = osd.cropped_pos_embed(table, 40, 72)
    assert cn.shape == (40 * 72, 64)
    for i, j in ((0, 0), (3, 61), (39, 71)):
        r, c = 172 + i, 156 + j
        for k in (1, 9):
            w = 1.0 / 10000 ** (k / 16.0)
            assert abs(float(cn[i * 72 + j, k]) - math.sin((c * 64 / 384) * w)) < 1e-6
            assert abs(float(cn[i * 72 + j, 32 + 16 + k]) - math.cos((r * 64 / 384) * w)) < 1e-6
    assert torch.allclose(pos_embed_crop(SD35Config(dim=64), 40, 72, "cpu"), cn, atol=1e-6)


def test_sd35_adaln_chunk_orders():
    """AdaLN-Zero: (shift, scale, gate, shift_mlp, scale_mlp, gate_mlp[, shift2, scale2, gate2]);
    AdaLN-Continuous: (scale, shift) (sd35_batch.py:351-393)."""
    D = 8
    p = {"n.linear.weight": torch.zeros(9 * D, D, dtype=D64),
         "n.linear.bias": torch.arange(9, dtype=D64).repeat_interleave(D) * 0.1,
         "c.linear.weight": torch.zeros(2 * D, D, dtype=D64),
         "c.linear.bias": torch.cat([torch.full((D,), 0.5), torch.full((D,), 0.25)]).double()}
    x = torch.randn(3, D, generator=g(20), dtype=D64)
    temb = torch.randn(D, generator=g(21), dtype=D64)
    a = osd.adaln_zero(p, "n", x, temb)
    nx = F.layer_norm(x, (D,), eps=1e-6)
    assert torch.allclose(a["normed"], nx * 1.1 + 0.0)
    assert torch.allclose(a["gate_msa"], torch.full((D,), 0.2, dtype=D64))
    assert torch.allclose(a["normed2"], nx * 1.7 + 0.6)
    assert torch.allclose(osd.adaln_continuous(p, "c", x, temb), nx * 1.5 + 0.25)


def test_sd35_joint_attention_layout_image_then_text():
    """Joint sequence = image tokens then text tokens (sd35_batch.py:444-484): the image
    rows of a library SDPA over cat([image, text]) are the image outputs."""
    from ditserve_amd.sd35 import SD35Config, random_state_dict
    cfg = SD35Config(dim=64, heads=1, head_dim=64, layers=2, dual_layers=(), text_dim=16, pooled_dim=16, ffn=128)
    p = {k: v.double() for k, v in random_state_dict(cfg, 0).items()}
    x_img = torch.randn(4, 64, generator=g(22), dtype=D64)
    x_txt = torch.randn(3, 64, generator=g(23), dtype=D64)
    pre = "transformer_blocks.0.attn"
    img, txt = osd.joint_attention(p, pre, x_img, x_txt, 1, False)

    def proj(x, n, norm=None):
        y = F.linear(x, p[f"{pre}.{n}.weight"], p[f"{pre}.{n}.bias"])
        return F.rms_norm(y, (64,), p[f"{pre}.{norm}.weight"], eps=1e-6) if norm else y
    q = torch.cat([proj(x_img, "to_q", "norm_q"), proj(x_txt, "add_q_proj", "norm_added_q")])
    k = torch.cat([proj(x_img, "to_k", "norm_k"), proj(x_txt, "add_k_proj", "norm_added_k")])
    v = torch.cat([proj(x_img, "to_v"), proj(x_txt, "add_v_proj")])
    o = F.scaled_dot_product_attention(q[None], k[None], v[None])[0]
    assert torch.allclose(img, F.linear(o[:4], p[f"{pre}.to_out.0.weight"], p[f"{pre}.to_out.0.bias"]), atol=1e-10)
    assert torch.allclose(txt, F.linear(o[4:], p[f"{pre}.to_add_out.weight"], p[f"{pre}.to_add_out.bias"]), atol=1e-10)


# ----------------------------------------------------------------- planted mistakes
def test_planted_rope_sign_error_is_caught(monkeypatch):
    """Rotating the wrong way passes norm preservation but fails the complex check."""
    orig = ow.apply_rotary

    def wrong(x, cos, sin):
        return orig(x, cos, -sin)
    monkeypatch.setattr(ow, "apply_rotary", wrong)
    with pytest.raises(AssertionError):
        test_apply_rotary_is_complex_multiplication()


def test_planted_dropped_gate_is_caught(monkeypatch):
    """A block that forgets the FFN gate fails the residual-structure check."""
    orig = ow.split_modulation

    def wrong(p, i, projected):
        parts = list(orig(p, i, projected))
        parts[5] = torch.ones_like(parts[5])
        return tuple(parts)
    monkeypatch.setattr(ow, "split_modulation", wrong)
    with pytest.raises(AssertionError):
        test_wan_block_residual_structure()


def _condition_embedder_variant(silu_before_proj=True, chunk_major=True):
    """The oracle's condition embedder with one of two plausible mistakes: no SiLU
    before time_proj, or the projection unflattened as (D, 6) instead of (6, D)."""
    def fn(p, t, text, freq_dim=256):
        pre = "condition_embedder"
        e = oc.timestep_embedding(t, freq_dim).to(text.dtype)
        temb = oc.linear(oc.silu(oc.linear(e, p[f"{pre}.time_embedder.linear_1.weight"],
                                           p[f"{pre}.time_embedder.linear_1.bias"])),
                         p[f"{pre}.time_embedder.linear_2.weight"], p[f"{pre}.time_embedder.linear_2.bias"])
        x = oc.silu(temb) if silu_before_proj else temb
        proj = oc.linear(x, p[f"{pre}.time_proj.weight"], p[f"{pre}.time_proj.bias"])
        proj = proj.unflatten(-1, (6, -1)) if chunk_major else proj.unflatten(-1, (-1, 6)).transpose(-1, -2)
        enc = oc.linear(oc.gelu_tanh(oc.linear(text, p[f"{pre}.text_embedder.linear_1.weight"],
                                               p[f"{pre}.text_embedder.linear_1.bias"])),
                        p[f"{pre}.text_embedder.linear_2.weight"], p[f"{pre}.text_embedder.linear_2.bias"])
        return temb, proj, enc
    return fn


def test_condition_embedder_variant_without_mistake_passes(monkeypatch):
    """The planted variants below differ from the oracle only by their mistake."""
    monkeypatch.setattr(ow, "condition_embedder", _condition_embedder_variant())
    test_condition_embedder_matches_module_composition()


@pytest.mark.parametrize("mistake", [dict(silu_before_proj=False), dict(chunk_major=False)],
                         ids=["no_silu_before_time_proj", "unflatten_d_by_6"])
def test_planted_condition_embedder_mistakes_are_caught(monkeypatch, mistake):
    monkeypatch.setattr(ow, "condition_embedder", _condition_embedder_variant(**mistake))
    with pytest.raises(AssertionError):
        test_condition_embedder_matches_module_composition()


def test_planted_adaln_continuous_order_error_is_caught(monkeypatch):
    def wrong(p, pre, x, temb, eps=1e-6):
        emb = oc.linear(oc.silu(temb), p[f"{pre}.linear.weight"], p[f"{pre}.linear.bias"])
        shift, scale = emb.reshape(2, -1).unbind(0)  # swapped
        return oc.layer_norm(x, eps) * (1.0 + scale) + shift
    monkeypatch.setattr(osd, "adaln_continuous", wrong)
    with pytest.raises(AssertionError):
        test_sd35_adaln_chunk_orders()

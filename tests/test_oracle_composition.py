"""Pin the oracle's attention and block compositions with cases whose answer the
mathematics fixes, computed here from library routines (F.linear, F.layer_norm,
F.gelu, F.conv2d) and scalar closed forms, never by calling the function under
test on other inputs:

* one key: softmax over a single key is 1, so attention returns that key's value
  row whatever q, k, the norms and RoPE are;
* zero q/k projections: every score is 0, so attention is the mean of the values;
* two tokens with q and k confined to one rotation pair: the scores, and so the
  softmax weights, follow in closed form from the norm weights, the RMS over the
  whole row and the rotation angle of that pair;
* a one-token Wan block with one text row (and an SD3.5 joint block with one image
  and one text token) reduces to linear maps, norms and the FFN.

The planted-mistake tests at the end show that a swapped k/v projection, swapped
q/k norm weights, RoPE applied to v, a swapped image/text output projection and a
dropped positional embedding each fail one of these checks.
"""
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


def _tiny_wan(seed=0):
    from ditserve_amd.wan import WanConfig, random_state_dict
    cfg = WanConfig(dim=256, heads=2, ffn=512, layers=1, text_dim=64)
    return cfg, {k: v.double() for k, v in random_state_dict(cfg, seed).items()}


def _lin(p, name, x):
    return F.linear(x, p[f"{name}.weight"], p[f"{name}.bias"])


def _zero_qk(p, pre, q="to_q", k="to_k"):
    p = dict(p)
    for n in (q, k):
        p[f"{pre}.{n}.weight"] = torch.zeros_like(p[f"{pre}.{n}.weight"])
        p[f"{pre}.{n}.bias"] = torch.zeros_like(p[f"{pre}.{n}.bias"])
    return p


# ------------------------------------------------------------ Wan self-attention
def test_wan_self_attention_single_key():
    """transformer_wan.py:50-69,138-156: with one token the output is to_out(to_v(x))."""
    _, p = _tiny_wan()
    pre = "blocks.0.attn1"
    x = torch.randn(1, 256, generator=g(1), dtype=D64)
    cos, sin = ow.rope_freqs((1, 1, 1))
    out = ow.self_attention(p, pre, x, cos, sin, 2)
    ref = _lin(p, f"{pre}.to_out.0", _lin(p, f"{pre}.to_v", x))
    assert torch.allclose(out, ref, atol=1e-12)


def test_wan_self_attention_uniform_when_q_k_vanish():
    """Zero to_q/to_k: q = k = 0 after RMSNorm, every score is 0 and each row is
    to_out(mean_j to_v(x_j)).  The grid has nonzero frame/row/column positions, so
    a rotation applied to v would change the mean."""
    _, p = _tiny_wan()
    pre = "blocks.0.attn1"
    p = _zero_qk(p, pre)
    grid = (2, 2, 3)
    x = torch.randn(12, 256, generator=g(2), dtype=D64)
    cos, sin = ow.rope_freqs(grid)
    out = ow.self_attention(p, pre, x, cos, sin, 2)
    ref = _lin(p, f"{pre}.to_out.0", _lin(p, f"{pre}.to_v", x).mean(0, keepdim=True)).expand(12, -1)
    assert torch.allclose(out, ref, atol=1e-12)


def _rot(theta, a, b):
    """(a + ib) e^{i theta}: the rotation of transformer_wan.py:183-186 written out."""
    return a * math.cos(theta) - b * math.sin(theta), a * math.sin(theta) + b * math.cos(theta)


def test_wan_self_attention_two_token_closed_form():
    """q and k confined, in head 0, to rotation pair 0 (bias-only projections).

    RMSNorm runs over the whole row of D = 256 values (norm_q / norm_k weights on
    their own tensor); the rest of q's energy sits in head 1 and the rest of k's in
    head 0's other pairs, so head 0's scores come from pair 0 alone (rotated by the
    token's frame index, theta^0 = 1) and stay small enough for the softmax not to
    saturate, and head 1's scores are all zero (uniform weights).
    """
    _, p = _tiny_wan()
    pre = "blocks.0.attn1"
    p = _zero_qk(p, pre)
    a1, a2, b1, b2, cq, ck = 0.7, -1.3, 0.4, 0.9, 1.0, 0.8
    bq = torch.zeros(256, dtype=D64)
    bq[:2] = torch.tensor([a1, a2], dtype=D64)
    bq[128:] = cq
    bk = torch.zeros(256, dtype=D64)
    bk[:2] = torch.tensor([b1, b2], dtype=D64)
    bk[2:128] = ck
    p[f"{pre}.to_q.bias"], p[f"{pre}.to_k.bias"] = bq, bk
    wq, wk = (1.5, 0.5), (0.8, 2.0)
    p[f"{pre}.norm_q.weight"] = p[f"{pre}.norm_q.weight"].clone()
    p[f"{pre}.norm_k.weight"] = p[f"{pre}.norm_k.weight"].clone()
    p[f"{pre}.norm_q.weight"][:2] = torch.tensor(wq, dtype=D64)
    p[f"{pre}.norm_k.weight"][:2] = torch.tensor(wk, dtype=D64)
    eps, D, dh = 1e-6, 256, 128
    rq = 1.0 / math.sqrt((a1 * a1 + a2 * a2 + 128 * cq * cq) / D + eps)
    rk = 1.0 / math.sqrt((b1 * b1 + b2 * b2 + 126 * ck * ck) / D + eps)
    qn = (wq[0] * a1 * rq, wq[1] * a2 * rq)
    kn = (wk[0] * b1 * rk, wk[1] * b2 * rk)
    frames = (0, 1)  # grid (2, 1, 1): token i sits at frame i
    x = torch.randn(2, 256, generator=g(3), dtype=D64)
    v = _lin(p, f"{pre}.to_v", x)
    o = torch.empty(2, 256, dtype=D64)
    for i in range(2):
        qi = _rot(frames[i], *qn)
        s = []
        for j in range(2):
            kj = _rot(frames[j], *kn)
            s.append((qi[0] * kj[0] + qi[1] * kj[1]) / math.sqrt(dh))
        m = max(s)
        e = [math.exp(t - m) for t in s]
        w = [t / sum(e) for t in e]
        assert 0.05 < w[0] < 0.95  # not saturated: the weights carry the scores
        o[i, :128] = w[0] * v[0, :128] + w[1] * v[1, :128]
        o[i, 128:] = 0.5 * (v[0, 128:] + v[1, 128:])
    ref = _lin(p, f"{pre}.to_out.0", o)
    cos, sin = ow.rope_freqs((2, 1, 1))
    out = ow.self_attention(p, pre, x, cos, sin, 2)
    assert torch.allclose(out, ref, atol=1e-10)


# ------------------------------------------------------------ Wan cross-attention
def test_wan_cross_attention_single_text_row():
    """transformer_wan.py:79-156: one text row -> every query gets to_out(to_v(enc))."""
    _, p = _tiny_wan()
    pre = "blocks.0.attn2"
    x = torch.randn(5, 256, generator=g(4), dtype=D64)
    enc = torch.randn(1, 256, generator=g(5), dtype=D64)
    out = ow.cross_attention(p, pre, x, enc, 2)
    ref = _lin(p, f"{pre}.to_out.0", _lin(p, f"{pre}.to_v", enc)).expand(5, -1)
    assert torch.allclose(out, ref, atol=1e-12)


def test_wan_cross_attention_uniform_and_zero_rows_attend():
    """Zero q/k: uniform weights over all 8 text rows, the 3 zero-padded rows
    included (no mask): to_out(mean_j to_v(enc_j)); to_v of a zero row is its bias."""
    _, p = _tiny_wan()
    pre = "blocks.0.attn2"
    p = _zero_qk(p, pre)
    x = torch.randn(4, 256, generator=g(6), dtype=D64)
    enc = torch.randn(8, 256, generator=g(7), dtype=D64)
    enc[5:] = 0
    out = ow.cross_attention(p, pre, x, enc, 2)
    ref = _lin(p, f"{pre}.to_out.0", _lin(p, f"{pre}.to_v", enc).mean(0, keepdim=True)).expand(4, -1)
    assert torch.allclose(out, ref, atol=1e-12)


# ------------------------------------------------------------ Wan block
def test_wan_block_one_token_one_text_row():
    """block.py:276-297 at S = 1, L = 1: both attentions reduce to to_out(to_v(.)),
    so the block is a chain of library LayerNorms, linear maps and the FFN with the
    chunk order shift, scale, gate, c_shift, c_scale, c_gate of _split_temb."""
    _, p = _tiny_wan()
    b = "blocks.0"
    h = torch.randn(1, 256, generator=g(8), dtype=D64)
    enc = torch.randn(1, 256, generator=g(9), dtype=D64)
    proj = torch.randn(6, 256, generator=g(10), dtype=D64) * 0.3
    cos, sin = ow.rope_freqs((1, 1, 1))
    out = ow.block_forward(p, 0, h, enc, proj, cos, sin, 2)
    sst = p[f"{b}.scale_shift_table"].reshape(6, 256)
    shift, scale, gate, c_shift, c_scale, c_gate = (sst + proj).unbind(0)
    n1 = F.layer_norm(h, (256,), eps=1e-6) * (1 + scale) + shift
    h1 = h + _lin(p, f"{b}.attn1.to_out.0", _lin(p, f"{b}.attn1.to_v", n1)) * gate
    h2 = h1 + _lin(p, f"{b}.attn2.to_out.0", _lin(p, f"{b}.attn2.to_v", enc))
    n3 = F.layer_norm(h2, (256,), eps=1e-6) * (1 + c_scale) + c_shift
    ff = _lin(p, f"{b}.ffn.net.2", F.gelu(_lin(p, f"{b}.ffn.net.0.proj", n3), approximate="tanh"))
    ref = h2 + ff * c_gate
    assert torch.allclose(out, ref, atol=1e-10)


def test_wan_block_packed_is_per_request_concatenation():
    """block_forward_packed over cu = [0, 4, 10]: each slice is its own block_forward."""
    _, p = _tiny_wan()
    h = torch.randn(10, 256, generator=g(11), dtype=D64)
    encs = [torch.randn(3, 256, generator=g(12 + i), dtype=D64) for i in range(2)]
    projs = torch.randn(2, 6, 256, generator=g(14), dtype=D64) * 0.1
    grids = [(1, 2, 2), (1, 2, 3)]
    rot = [ow.rope_freqs(gr) for gr in grids]
    out = ow.block_forward_packed(p, 0, h, [0, 4, 10], encs, projs, rot, 2)
    for m, (s0, s1) in enumerate(((0, 4), (4, 10))):
        solo = ow.block_forward(p, 0, h[s0:s1], encs[m], projs[m], rot[m][0], rot[m][1], 2)
        assert torch.equal(out[s0:s1], solo)


def test_wan_forward_without_blocks_is_conv3d_then_prediction():
    """forward() with no blocks = patch embedding (a library Conv3d) then norm_out,
    proj_out and the unpatchify index map (element-wise), t only entering through temb."""
    cfg, p = _tiny_wan()
    ocfg = dict(patch=(1, 2, 2), head_dim=128, heads=2, layers=1, freq_dim=256, eps=1e-6, out_ch=16)
    lat = torch.randn(16, 2, 4, 6, generator=g(15), dtype=D64)
    text = torch.randn(4, 64, generator=g(16), dtype=D64)
    out = ow.forward(p, ocfg, lat, 300.0, text, blocks=0)
    hid = F.conv3d(lat[None], p["patch_embedding.weight"], p["patch_embedding.bias"], stride=(1, 2, 2))
    hid = hid.flatten(2)[0].t()  # [S, D], token order f, h, w
    temb, _, _ = ow.condition_embedder(p, torch.tensor([300.0]), text)
    shift, scale = (p["scale_shift_table"].reshape(2, -1) + temb).unbind(0)
    y = _lin(p, "proj_out", F.layer_norm(hid, (256,), eps=1e-6) * (1 + scale) + shift)
    for c, f, hh, ww in ((0, 0, 0, 0), (5, 1, 3, 4), (15, 1, 2, 5), (7, 0, 1, 3)):
        tok = (f * 2 + hh // 2) * 3 + ww // 2
        feat = ((hh % 2) * 2 + ww % 2) * 16 + c
        assert abs(float(out[c, f, hh, ww]) - float(y[tok, feat])) < 1e-10


def test_wan_model_timestep_and_cfg_combine():
    """runtime.py:153-163: Wan2.1 gives [B]; Wan2.2 gives [B, F*(H/2)*(W/2)], all equal.
    block.py:483: g = 1 returns cond, g = 0 returns uncond, and the map is affine in g."""
    a = ow.model_timestep((2, 16, 3, 8, 10), 700.0, False)
    b = ow.model_timestep((2, 48, 3, 8, 10), 700.0, True)
    assert a.shape == (2,) and bool((a == 700.0).all())
    assert b.shape == (2, 3 * 4 * 5) and bool((b == 700.0).all())
    c, u = torch.randn(5, generator=g(17), dtype=D64), torch.randn(5, generator=g(18), dtype=D64)
    assert torch.allclose(ow.cfg_combine(c, u, 1.0), c, atol=1e-15) and torch.equal(ow.cfg_combine(c, u, 0.0), u)
    g3, g5 = ow.cfg_combine(c, u, 3.0), ow.cfg_combine(c, u, 5.0)
    assert torch.allclose(g5 - g3, 2.0 * (c - u), atol=1e-14)


def test_wan_block_flops_matches_counted_work():
    """9.4327e12 FLOP per block-forward at S = 32760 (D = 1536, FFN 8960, L = 512):
    4 D x D projections and 2 text projections, 4 S^2 D, 4 S L D and 4 S D F."""
    s, d, f, l = 32760, 1536, 8960, 512
    got = ow.block_flops(s, d, 12, f, l)
    assert got == 2 * s * d * d * 6 + 2 * l * d * d * 2 + 4 * s * s * d + 4 * s * l * d + 4 * s * d * f
    assert abs(got / 9.4327e12 - 1) < 1e-4


# ------------------------------------------------------------ SD3.5
def _tiny_sd35(seed=0, layers=2, dual=()):
    from ditserve_amd.sd35 import SD35Config, random_state_dict
    cfg = SD35Config(dim=128, heads=2, head_dim=64, layers=layers, dual_layers=dual, text_dim=32, pooled_dim=24,
                     ffn=256)
    return cfg, {k: v.double() for k, v in random_state_dict(cfg, seed).items()}


def test_sd35_joint_attention_single_image_token_no_text():
    """sd35_batch.py:681-694 dual attention on one image token: to_out(to_v(x))."""
    _, p = _tiny_sd35()
    pre = "transformer_blocks.0.attn"
    x = torch.randn(1, 128, generator=g(20), dtype=D64)
    out = osd.self_attention(p, pre, x, 2)
    assert torch.allclose(out, _lin(p, f"{pre}.to_out.0", _lin(p, f"{pre}.to_v", x)), atol=1e-12)


def test_sd35_joint_attention_uniform_pairs_projections():
    """Zero image and text q/k projections: every joint row averages the values of
    the segment's image rows (to_v) and text rows (add_v_proj); image rows leave
    through to_out, text rows through to_add_out (sd35_batch.py:410-495)."""
    _, p = _tiny_sd35()
    pre = "transformer_blocks.0.attn"
    p = _zero_qk(_zero_qk(p, pre), pre, "add_q_proj", "add_k_proj")
    xi = torch.randn(3, 128, generator=g(21), dtype=D64)
    xt = torch.randn(2, 128, generator=g(22), dtype=D64)
    img, txt = osd.joint_attention(p, pre, xi, xt, 2, False)
    mean_v = torch.cat([_lin(p, f"{pre}.to_v", xi), _lin(p, f"{pre}.add_v_proj", xt)]).mean(0, keepdim=True)
    assert torch.allclose(img, _lin(p, f"{pre}.to_out.0", mean_v).expand(3, -1), atol=1e-12)
    assert torch.allclose(txt, _lin(p, f"{pre}.to_add_out", mean_v).expand(2, -1), atol=1e-12)
    img2, txt2 = osd.joint_attention(p, pre, xi, xt, 2, True)  # context_pre_only: no text output
    assert txt2 is None and torch.allclose(img2, img, atol=0)


def test_sd35_patch_embed_matches_conv2d_plus_crop():
    """PatchEmbed: Conv2d(k = s = 2) on the latent, flattened row-major, plus the
    centre crop of the sin-cos table (whose values the closed-form test pins)."""
    _, p = _tiny_sd35()
    table = osd.pos_embed_table(128, max_size=384, base_size=64)
    lat = torch.randn(16, 6, 10, generator=g(23), dtype=D64)
    out = osd.patch_embed(p, lat, table.double(), 2)
    conv = F.conv2d(lat[None], p["pos_embed.proj.weight"], p["pos_embed.proj.bias"], stride=2)[0]
    conv = conv.flatten(1).t()  # [3*5, D]
    top, left = (384 - 3) // 2, (384 - 5) // 2
    for r in range(3):
        for c in range(5):
            ref = conv[r * 5 + c] + table[(top + r) * 384 + left + c].double()
            assert torch.allclose(out[r * 5 + c], ref, atol=1e-12)


def test_sd35_time_text_embed_matches_module_composition():
    """CombinedTimestepTextProjEmbeddings: TimestepEmbedding(Timesteps(256)) +
    PixArtAlphaTextProjection(pooled), each Linear-SiLU-Linear."""
    _, p = _tiny_sd35()
    pre = "time_text_embed"

    def seq(a, b, din):
        m = torch.nn.Sequential(torch.nn.Linear(din, 128), torch.nn.SiLU(), torch.nn.Linear(128, 128)).double()
        m[0].weight.data, m[0].bias.data = p[f"{pre}.{a}.weight"], p[f"{pre}.{a}.bias"]
        m[2].weight.data, m[2].bias.data = p[f"{pre}.{b}.weight"], p[f"{pre}.{b}.bias"]
        return m
    te = seq("timestep_embedder.linear_1", "timestep_embedder.linear_2", 256)
    tx = seq("text_embedder.linear_1", "text_embedder.linear_2", 24)
    t = torch.tensor([0.0, 421.0])
    pooled = torch.randn(2, 24, generator=g(24), dtype=D64)
    with torch.no_grad():
        ref = te(oc.timestep_embedding(t, 256).double()) + tx(pooled)
    assert torch.allclose(osd.time_text_embed(p, t, pooled), ref, atol=1e-12)


def test_sd35_ffn_matches_module_composition():
    _, p = _tiny_sd35()
    pre = "transformer_blocks.0.ff"
    m = torch.nn.Sequential(torch.nn.Linear(128, 256), torch.nn.GELU(approximate="tanh"),
                            torch.nn.Linear(256, 128)).double()
    m[0].weight.data, m[0].bias.data = p[f"{pre}.net.0.proj.weight"], p[f"{pre}.net.0.proj.bias"]
    m[2].weight.data, m[2].bias.data = p[f"{pre}.net.2.weight"], p[f"{pre}.net.2.bias"]
    x = torch.randn(3, 128, generator=g(25), dtype=D64)
    with torch.no_grad():
        assert torch.allclose(osd.ffn(p, pre, x), m(x), atol=1e-12)


def test_sd35_joint_block_one_image_one_text_token_uniform():
    """A joint block on one image and one text token with zero q/k projections
    (uniform weights over the 2 joint rows) reduces to library norms, linear maps and
    FFNs with the AdaLN-Zero chunk order (sd35_batch.py:336-376,647-708)."""
    cfg, p = _tiny_sd35()
    pre = "transformer_blocks.0"
    p = _zero_qk(_zero_qk(p, f"{pre}.attn"), f"{pre}.attn", "add_q_proj", "add_k_proj")
    ocfg = dict(heads=2, eps=1e-6, layers=2, dual_layers=())
    h = torch.randn(1, 128, generator=g(26), dtype=D64)
    c = torch.randn(1, 128, generator=g(27), dtype=D64)
    temb = torch.randn(128, generator=g(28), dtype=D64)
    oh, oc_ = osd.joint_block(p, 0, h, c, temb, ocfg)

    def chunks(name):
        return _lin(p, f"{pre}.{name}.linear", F.silu(temb)).reshape(6, 128).unbind(0)
    sh, sc, ga, shm, scm, gam = chunks("norm1")
    csh, csc, cga, cshm, cscm, cgam = chunks("norm1_context")
    ln = lambda x: F.layer_norm(x, (128,), eps=1e-6)  # noqa: E731
    ni, nt = ln(h) * (1 + sc) + sh, ln(c) * (1 + csc) + csh
    mean_v = 0.5 * (_lin(p, f"{pre}.attn.to_v", ni) + _lin(p, f"{pre}.attn.add_v_proj", nt))
    h1 = h + ga * _lin(p, f"{pre}.attn.to_out.0", mean_v)
    c1 = c + cga * _lin(p, f"{pre}.attn.to_add_out", mean_v)

    def ff(name, x):
        return _lin(p, f"{pre}.{name}.net.2", F.gelu(_lin(p, f"{pre}.{name}.net.0.proj", x), approximate="tanh"))
    h2 = h1 + gam * ff("ff", ln(h1) * (1 + scm) + shm)
    c2 = c1 + cgam * ff("ff_context", ln(c1) * (1 + cscm) + cshm)
    assert torch.allclose(oh, h2, atol=1e-10) and torch.allclose(oc_, c2, atol=1e-10)


def _one_token_inputs(seed):
    h = torch.randn(1, 128, generator=g(seed), dtype=D64)
    c = torch.randn(1, 128, generator=g(seed + 1), dtype=D64)
    temb = torch.randn(128, generator=g(seed + 2), dtype=D64) * 4.0  # gates of order 1
    return h, c, temb


def _ff(p, pre, x):
    return _lin(p, f"{pre}.net.2", F.gelu(_lin(p, f"{pre}.net.0.proj", x), approximate="tanh"))


def _ln128(x):
    return F.layer_norm(x, (128,), eps=1e-6)


def test_sd35_dual_block_one_image_one_text_token():
    """A dual-attention block (sd35_batch.py:647-708 with use_dual_attention): norm1's
    9-chunk AdaLN-Zero is (shift, scale, gate, shift_mlp, scale_mlp, gate_mlp, shift2,
    scale2, gate2) (sd35_batch.py:351-363); normed2 = LN(h)(1 + scale2) + shift2 of the
    PRE-attention h; attn2 over one image token is to_out(to_v(normed2)) whatever its q/k;
    its term gate2 · attn2 is added after the joint residual and before the image FFN,
    whose LayerNorm reads the updated h (sd35_batch.py:681-699)."""
    _, p = _tiny_sd35(dual=(0,))
    pre = "transformer_blocks.0"
    p = _zero_qk(_zero_qk(p, f"{pre}.attn"), f"{pre}.attn", "add_q_proj", "add_k_proj")
    ocfg = dict(heads=2, eps=1e-6, layers=2, dual_layers=(0,))
    h, c, temb = _one_token_inputs(40)
    oh, oc_ = osd.joint_block(p, 0, h, c, temb, ocfg)
    sh, sc, ga, shm, scm, gam, sh2, sc2, ga2 = _lin(p, f"{pre}.norm1.linear", F.silu(temb)).reshape(9, 128).unbind(0)
    csh, csc, cga, cshm, cscm, cgam = _lin(p, f"{pre}.norm1_context.linear", F.silu(temb)).reshape(6, 128).unbind(0)
    ni, nt = _ln128(h) * (1 + sc) + sh, _ln128(c) * (1 + csc) + csh
    ni2 = _ln128(h) * (1 + sc2) + sh2
    mean_v = 0.5 * (_lin(p, f"{pre}.attn.to_v", ni) + _lin(p, f"{pre}.attn.add_v_proj", nt))
    h1 = h + ga * _lin(p, f"{pre}.attn.to_out.0", mean_v)
    h1 = h1 + ga2 * _lin(p, f"{pre}.attn2.to_out.0", _lin(p, f"{pre}.attn2.to_v", ni2))
    h2 = h1 + gam * _ff(p, f"{pre}.ff", _ln128(h1) * (1 + scm) + shm)
    c1 = c + cga * _lin(p, f"{pre}.attn.to_add_out", mean_v)
    c2 = c1 + cgam * _ff(p, f"{pre}.ff_context", _ln128(c1) * (1 + cscm) + cshm)
    assert torch.allclose(oh, h2, atol=1e-10) and torch.allclose(oc_, c2, atol=1e-10)


def test_sd35_last_block_one_image_one_text_token():
    """The last (context_pre_only) block: the text goes through AdaLN-Continuous,
    (scale, shift) = chunk(2) (sd35_batch.py:379-393, 624-628), into the joint attention,
    which returns no text output; only the image stream gets its gated residual and FFN,
    and the block returns no text (sd35_batch.py:666-708)."""
    _, p = _tiny_sd35()
    pre = "transformer_blocks.1"
    p = _zero_qk(_zero_qk(p, f"{pre}.attn"), f"{pre}.attn", "add_q_proj", "add_k_proj")
    ocfg = dict(heads=2, eps=1e-6, layers=2, dual_layers=())
    h, c, temb = _one_token_inputs(43)
    oh, oc_ = osd.joint_block(p, 1, h, c, temb, ocfg)
    assert oc_ is None
    sh, sc, ga, shm, scm, gam = _lin(p, f"{pre}.norm1.linear", F.silu(temb)).reshape(6, 128).unbind(0)
    cscale, cshift = _lin(p, f"{pre}.norm1_context.linear", F.silu(temb)).reshape(2, 128).unbind(0)
    ni, nt = _ln128(h) * (1 + sc) + sh, _ln128(c) * (1 + cscale) + cshift
    mean_v = 0.5 * (_lin(p, f"{pre}.attn.to_v", ni) + _lin(p, f"{pre}.attn.add_v_proj", nt))
    h1 = h + ga * _lin(p, f"{pre}.attn.to_out.0", mean_v)
    h2 = h1 + gam * _ff(p, f"{pre}.ff", _ln128(h1) * (1 + scm) + shm)
    assert torch.allclose(oh, h2, atol=1e-10)


def _joint_block_variant(dual_gate_chunk=8, normed2_from_pre=True, dual_before_ffn=True, last_text="continuous"):
    """The oracle's joint block written out with switches for plausible mistakes:
    the dual gate read from another chunk (2 = gate_msa, 5 = gate_mlp), normed2 taken
    from the post-attention h, the dual term added after the FFN, and the last block's
    text normalised in AdaLN-Zero's chunk order (shift first) or not modulated at all."""
    def fn(p, i, h, c, temb, cfg, attn=oc.sdpa):
        pre = f"transformer_blocks.{i}"
        heads, eps = cfg["heads"], cfg["eps"]
        pre_only, dual = i == cfg["layers"] - 1, i in cfg["dual_layers"]
        d = h.shape[-1]
        ch = oc.linear(oc.silu(temb), p[f"{pre}.norm1.linear.weight"], p[f"{pre}.norm1.linear.bias"]).reshape(-1, d)
        normed = oc.layer_norm(h, eps) * (1.0 + ch[1]) + ch[0]
        cc = oc.linear(oc.silu(temb), p[f"{pre}.norm1_context.linear.weight"],
                       p[f"{pre}.norm1_context.linear.bias"]).reshape(-1, d)
        if pre_only:
            if last_text == "continuous":
                nc = oc.layer_norm(c, eps) * (1.0 + cc[0]) + cc[1]
            elif last_text == "zero_order":
                nc = oc.layer_norm(c, eps) * (1.0 + cc[1]) + cc[0]
            else:
                nc = oc.layer_norm(c, eps)
        else:
            nc = oc.layer_norm(c, eps) * (1.0 + cc[1]) + cc[0]
        img, txt = osd.joint_attention(p, f"{pre}.attn", normed, nc, heads, pre_only, eps, attn)
        h_pre = h
        h = h + ch[2] * img

        def dual_term(hh):
            src = h_pre if normed2_from_pre else hh
            n2 = oc.layer_norm(src, eps) * (1.0 + ch[7]) + ch[6]
            return ch[dual_gate_chunk] * osd.self_attention(p, f"{pre}.attn2", n2, heads, eps, attn)
        if dual and dual_before_ffn:
            h = h + dual_term(h)
        h = h + ch[5] * osd.ffn(p, f"{pre}.ff", oc.layer_norm(h, eps) * (1.0 + ch[4]) + ch[3])
        if dual and not dual_before_ffn:
            h = h + dual_term(h)
        if pre_only:
            return h, None
        c = c + cc[2] * txt
        c = c + cc[5] * osd.ffn(p, f"{pre}.ff_context", oc.layer_norm(c, eps) * (1.0 + cc[4]) + cc[3])
        return h, c
    return fn


def test_joint_block_variant_without_mistake_passes(monkeypatch):
    """The planted variants below differ from the oracle only by their mistake."""
    monkeypatch.setattr(osd, "joint_block", _joint_block_variant())
    test_sd35_dual_block_one_image_one_text_token()
    test_sd35_last_block_one_image_one_text_token()
    test_sd35_joint_block_one_image_one_text_token_uniform()


@pytest.mark.parametrize("mistake,test", [
    (dict(dual_gate_chunk=2), "dual"), (dict(dual_gate_chunk=5), "dual"),
    (dict(normed2_from_pre=False), "dual"), (dict(dual_before_ffn=False), "dual"),
    (dict(last_text="zero_order"), "last"), (dict(last_text="plain"), "last")],
    ids=["dual_gate_is_gate_msa", "dual_gate_from_chunk5", "normed2_after_attention", "dual_after_ffn",
         "last_block_adaln_zero_order", "last_block_text_unmodulated"])
def test_planted_joint_block_mistakes_are_caught(monkeypatch, mistake, test):
    monkeypatch.setattr(osd, "joint_block", _joint_block_variant(**mistake))
    check = test_sd35_dual_block_one_image_one_text_token if test == "dual" else test_sd35_last_block_one_image_one_text_token
    with pytest.raises(AssertionError):
        check()


def test_sd35_forward_without_blocks_is_patch_embed_then_output():
    """forward() with no blocks = PatchEmbed (a library Conv2d plus the pinned table
    crop), AdaLayerNormContinuous (scale first, sd35_batch.py:379-393), proj_out and the
    unpatchify index map (element-wise): output channel c of pixel (2r + i, 2q + j) is
    feature (i * 2 + j) * C + c of token r * W' + q; the text only enters through blocks."""
    cfg, p = _tiny_sd35()
    ocfg = dict(dim=128, pos_max=384, base_size=64, patch=2, layers=0, eps=1e-6, out_ch=16, heads=2,
                dual_layers=())
    lat = torch.randn(16, 6, 10, generator=g(29), dtype=D64)
    text = torch.randn(3, 32, generator=g(30), dtype=D64)
    pooled = torch.randn(24, generator=g(31), dtype=D64)
    table = osd.pos_embed_table(128, max_size=384, base_size=64).double()
    out = osd.forward(p, ocfg, lat, 250.0, text, pooled, table=table)
    conv = F.conv2d(lat[None], p["pos_embed.proj.weight"], p["pos_embed.proj.bias"], stride=2)[0]
    hid = conv.flatten(1).t()  # [3*5, D], token order row-major over the patch grid
    top, left = (384 - 3) // 2, (384 - 5) // 2
    hid = hid + torch.stack([table[(top + r) * 384 + left + q] for r in range(3) for q in range(5)])
    temb = osd.time_text_embed(p, torch.tensor([250.0]), pooled[None])[0]
    scale, shift = _lin(p, "norm_out.linear", F.silu(temb)).reshape(2, -1).unbind(0)
    y = _lin(p, "proj_out", F.layer_norm(hid, (128,), eps=1e-6) * (1 + scale) + shift)
    for c, hh, ww in ((0, 0, 0), (5, 3, 4), (15, 5, 9), (7, 2, 7), (11, 4, 1)):
        tok = (hh // 2) * 5 + ww // 2
        feat = ((hh % 2) * 2 + ww % 2) * 16 + c
        assert abs(float(out[c, hh, ww]) - float(y[tok, feat])) < 1e-10
    other = osd.forward(p, ocfg, lat, 250.0, torch.zeros_like(text), pooled, table=table)
    assert torch.equal(out, other)
    assert all(torch.equal(a, b) for a, b in zip(
        osd.forward_packed(p, ocfg, [lat, lat[:, :4, :6]], [250.0, 10.0], [text, text[:2]], [pooled, -pooled]),
        [out, osd.forward(p, ocfg, lat[:, :4, :6], 10.0, text[:2], -pooled, table=table)]))


def test_planted_unpatchify_transpose_is_caught(monkeypatch):
    """An SD3.5 output map with the patch-internal row and column swapped fails the
    element-wise unpatchify check."""
    orig = osd.forward

    def wrong(p, cfg, latent, t, text, pooled, attn=oc.sdpa, table=None):
        out = orig(p, cfg, latent, t, text, pooled, attn, table)
        c, h, w = out.shape
        return out.reshape(c, h // 2, 2, w // 2, 2).transpose(2, 4).reshape(c, h, w)
    _planted(monkeypatch, osd, "forward", wrong)
    with pytest.raises(AssertionError):
        test_sd35_forward_without_blocks_is_patch_embed_then_output()


# ------------------------------------------------------------ planted mistakes
def _planted(monkeypatch, module, name, wrong):
    monkeypatch.setattr(module, name, wrong)


def test_planted_kv_swap_is_caught(monkeypatch):
    orig = ow.self_attention

    def wrong(p, pre, x, *a, **k):
        q = dict(p)
        q[f"{pre}.to_k.weight"], q[f"{pre}.to_v.weight"] = p[f"{pre}.to_v.weight"], p[f"{pre}.to_k.weight"]
        q[f"{pre}.to_k.bias"], q[f"{pre}.to_v.bias"] = p[f"{pre}.to_v.bias"], p[f"{pre}.to_k.bias"]
        return orig(q, pre, x, *a, **k)
    _planted(monkeypatch, ow, "self_attention", wrong)
    with pytest.raises(AssertionError):
        test_wan_self_attention_single_key()
    with pytest.raises(AssertionError):
        test_wan_self_attention_uniform_when_q_k_vanish()


def test_planted_norm_weight_swap_is_caught(monkeypatch):
    """norm_k's weight applied to q (and norm_q's to k): invisible without RoPE,
    caught by the rotated two-token closed form."""
    orig = ow.qk_norm_rope

    def wrong(q, k, wq, wk, cos, sin, heads, eps=1e-6):
        return orig(q, k, wk, wq, cos, sin, heads, eps)
    _planted(monkeypatch, ow, "qk_norm_rope", wrong)
    with pytest.raises(AssertionError):
        test_wan_self_attention_two_token_closed_form()


def test_planted_rope_on_v_is_caught(monkeypatch):
    orig_linear = ow.linear

    def wrong_self_attention(p, pre, x, cos, sin, heads, eps=1e-6, attn=oc.sdpa):
        def lin(xx, w, b=None):
            y = orig_linear(xx, w, b)
            if w is p[f"{pre}.to_v.weight"]:
                y = ow.apply_rotary(y.unflatten(-1, (heads, -1)), cos, sin).flatten(1)
            return y
        monkeypatch.setattr(ow, "linear", lin)
        try:
            return orig_self_attention(p, pre, x, cos, sin, heads, eps, attn)
        finally:
            monkeypatch.setattr(ow, "linear", orig_linear)
    orig_self_attention = ow.self_attention
    _planted(monkeypatch, ow, "self_attention", wrong_self_attention)
    with pytest.raises(AssertionError):
        test_wan_self_attention_uniform_when_q_k_vanish()


def test_planted_output_projection_swap_is_caught(monkeypatch):
    """Image rows leaving through to_add_out (and text rows through to_out)."""
    orig = osd.joint_attention

    def wrong(p, pre, x_img, x_txt, heads, context_pre_only, eps=1e-6, attn=oc.sdpa):
        q = dict(p)
        for s in ("weight", "bias"):
            q[f"{pre}.to_out.0.{s}"], q[f"{pre}.to_add_out.{s}"] = p[f"{pre}.to_add_out.{s}"], p[f"{pre}.to_out.0.{s}"]
        return orig(q, pre, x_img, x_txt, heads, context_pre_only, eps, attn)
    _planted(monkeypatch, osd, "joint_attention", wrong)
    with pytest.raises(AssertionError):
        test_sd35_joint_attention_uniform_pairs_projections()


def test_planted_missing_pos_embed_is_caught(monkeypatch):
    orig = osd.patch_embed

    def wrong(p, latent, table, patch=2):
        return orig(p, latent, torch.zeros_like(table), patch)
    _planted(monkeypatch, osd, "patch_embed", wrong)
    with pytest.raises(AssertionError):
        test_sd35_patch_embed_matches_conv2d_plus_crop()

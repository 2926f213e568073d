"""Seeded sweeps of random shapes inside each kernel's documented limits, against the
oracle's formulas evaluated in fp32 on the GPU (the same bf16-rounded inputs).

* GEMM: M in [1, 5000], N % 8 == 0 up to 5000, K % 32 == 0 up to 4096, every epilogue,
  A as a column slice of a wider buffer (lda > K) for some cases, gated residuals over
  random segment tables.  cos >= 0.99999, relative L2 <= 5e-3 (bf16 output rounding).
* Varlen attention: 1-5 segments of 0-900 queries and 0-900 keys (segments without
  queries or without keys included), 1-4 heads of 64 or 128, plain and pre-scaled q.
  Rows of a segment without keys are zero.  cos >= 0.9999, relative L2 <= 1e-2.
* Joint attention from two sources: 1-4 segments of 0-700 image and 0-400 text rows.
* AdaLN (LayerNorm / RMSNorm, modulated over random segments or affine) and per-head
  or across-head QK RMSNorm at random T and D <= 6144.
The shapes are drawn once from a fixed seed (segment cuts per case from its own
seed) and printed with each case."""
import math
import random

import pytest
import torch

from oracle import common as oc

pytestmark = pytest.mark.gpu
DEV = "cuda"
RNG = random.Random(20261202)


def _ops():
    from ditserve_amd import ops
    return ops


def _g(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


def _bf(x):
    return x.to(torch.bfloat16).float()


def _metrics(got, ref):
    g, r = got.double().reshape(-1), ref.double().reshape(-1)
    return float(torch.nn.functional.cosine_similarity(g, r, dim=0)), float((g - r).norm() / r.norm().clamp_min(1e-30))


def _cu(lengths):
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    return cu


GEMM_RANDOM = []
for _ in range(24):
    GEMM_RANDOM.append((RNG.randint(1, 5000), 8 * RNG.randint(1, 625), 32 * RNG.randint(1, 128),
                        RNG.choice(["bias", "gelu", "f32", "silu", "gate_res", "res"]), RNG.random() < 0.3))


@pytest.mark.parametrize("M,N,K,epi,sliced", GEMM_RANDOM)
def test_gemm_random_shapes(M, N, K, epi, sliced):
    ops = _ops()
    g = _g(M * 7 + N * 3 + K)
    base = torch.randn((M, K + (64 if sliced else 0)), generator=g, device=DEV).bfloat16()
    a = base[:, 32:32 + K] if sliced else base
    w = (torch.randn((N, K), generator=g, device=DEV) * 0.02).bfloat16()
    b = torch.randn((N,), generator=g, device=DEV) * 0.1
    kw, ref_extra, rng = {}, None, random.Random(M * 31 + N * 7 + K)
    y = oc.linear(a.float(), w.float(), b)
    if epi in ("gate_res", "res"):
        r = torch.randn((M, N), generator=g, device=DEV).bfloat16()
        kw["residual"] = r
        if epi == "gate_res":
            nseg = rng.randint(1, 4) if M >= 4 else 1
            cuts = sorted(rng.sample(range(1, M), nseg - 1)) if nseg > 1 else []
            cu = [0, *cuts, M]
            gate = torch.randn((len(cu) - 1, N), generator=g, device=DEV)
            kw.update(gate=gate, segments=ops.Segments(cu, DEV))
            gt = torch.cat([gate[i].expand(cu[i + 1] - cu[i], N) for i in range(len(cu) - 1)])
            ref_extra = r.float() + _bf(y) * gt
        else:
            ref_extra = r.float() + _bf(y)
    out = ops.linear(a, w, b, epi, **kw).float()
    if ref_extra is not None:
        ref = ref_extra
    elif epi == "gelu":
        ref = oc.gelu_tanh(y)
    elif epi == "silu":
        ref = oc.silu(y)
    else:
        ref = y
    cos, rel = _metrics(out, ref)
    print(f"gemm {M}x{N}x{K} {epi} sliced={sliced}: cos {cos:.7f} rel {rel:.2e}")
    assert torch.isfinite(out).all() and cos >= 0.99999 and rel <= 5e-3


ATTN_RANDOM = []
for _ in range(16):
    nseg = RNG.randint(1, 5)
    lq = [RNG.randint(1, 900) if RNG.random() < 0.75 else 0 for _ in range(nseg)]
    lk = [RNG.randint(1, 900) if RNG.random() < 0.75 else 0 for _ in range(nseg)]
    if not any(a and b for a, b in zip(lq, lk)):  # at least one segment with queries and keys
        lq[0], lk[0] = RNG.randint(1, 900), RNG.randint(1, 900)
    ATTN_RANDOM.append((tuple(lq), tuple(lk), RNG.randint(1, 4), RNG.choice([64, 128]), RNG.random() < 0.5))


@pytest.mark.parametrize("lq,lk,heads,hd,pre", ATTN_RANDOM)
def test_attention_random_segment_tables(lq, lk, heads, hd, pre):
    ops = _ops()
    cu_q, cu_k = _cu(lq), _cu(lk)
    Tq, Tk, W = cu_q[-1], cu_k[-1], heads * hd
    g = _g(Tq * 13 + Tk * 7 + heads * 3 + hd)
    q = torch.randn((Tq, W), generator=g, device=DEV).bfloat16()
    k = torch.randn((Tk, W), generator=g, device=DEV).bfloat16()
    v = torch.randn((Tk, W), generator=g, device=DEV).bfloat16()
    seg_q, seg_k = ops.Segments(cu_q, DEV), ops.Segments(cu_k, DEV)
    if pre:
        qp = (q.float() * (ops.LOG2E / math.sqrt(hd))).bfloat16()
        out = ops.flash_attn_varlen(qp, k, v, seg_q, seg_k, heads, hd, q_prescaled=True).float()
        # the reference sees the pre-scaled q's own rounding: scores = qp.k / log2(e)
        q_ref, scale = qp.float() / ops.LOG2E, 1.0
    else:
        out = ops.flash_attn_varlen(q, k, v, seg_q, seg_k, heads, hd).float()
        q_ref, scale = q.float(), 1.0 / math.sqrt(hd)
    ref = torch.zeros((Tq, W), device=DEV)
    for m in range(len(lq)):
        q0, q1, k0, k1 = cu_q[m], cu_q[m + 1], cu_k[m], cu_k[m + 1]
        if q1 == q0 or k1 == k0:
            continue
        qs = q_ref[q0:q1].view(-1, heads, hd).transpose(0, 1)
        ks = k[k0:k1].float().view(-1, heads, hd).transpose(0, 1)
        vs = v[k0:k1].float().view(-1, heads, hd).transpose(0, 1)
        p = torch.softmax(torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale, dim=-1)
        ref[q0:q1] = torch.matmul(p, vs).transpose(0, 1).reshape(q1 - q0, W)
    for m in range(len(lq)):
        if lk[m] == 0:
            assert torch.equal(out[cu_q[m]:cu_q[m + 1]], torch.zeros_like(out[cu_q[m]:cu_q[m + 1]]))
    cos, rel = _metrics(out, ref)
    print(f"attention q{lq} k{lk} heads {heads} hd {hd} pre={pre}: cos {cos:.6f} rel {rel:.2e}")
    assert torch.isfinite(out).all() and cos >= 0.9999 and rel <= 1e-2


JOINT_RANDOM = []
for _ in range(10):
    nseg = RNG.randint(1, 4)
    li = [RNG.randint(1, 700) if RNG.random() < 0.8 else 0 for _ in range(nseg)]
    lt = [RNG.randint(1, 400) if RNG.random() < 0.8 else 0 for _ in range(nseg)]
    li[0], lt[-1] = li[0] or RNG.randint(1, 700), lt[-1] or RNG.randint(1, 400)  # both sources non-empty
    JOINT_RANDOM.append((tuple(li), tuple(lt), RNG.randint(1, 4)))


@pytest.mark.parametrize("li,lt,heads", JOINT_RANDOM)
def test_joint_attention_random_layouts(li, lt, heads):
    """Joint attention read in place from the image and text projections (head_dim 64,
    q pre-scaled): segment m attends over its image rows followed by its text rows; the
    image/text seam falls at every offset the random lengths give."""
    ops = _ops()
    hd, W = 64, heads * 64
    cu_i, cu_t = _cu(li), _cu(lt)
    cu_j = [a + b for a, b in zip(cu_i, cu_t)]
    seg_i, seg_t, seg_j = ops.Segments(cu_i, DEV), ops.Segments(cu_t, DEV), ops.Segments(cu_j, DEV)
    g = _g(cu_i[-1] * 5 + cu_t[-1] * 3 + heads)
    qkv_i = torch.randn((cu_i[-1], 3 * W), generator=g, device=DEV).bfloat16()
    qkv_t = torch.randn((cu_t[-1], 3 * W), generator=g, device=DEV).bfloat16()
    scale = ops.LOG2E / math.sqrt(hd)
    qkv_i[:, :W] = (qkv_i[:, :W].float() * scale).bfloat16()
    qkv_t[:, :W] = (qkv_t[:, :W].float() * scale).bfloat16()
    vt = ops.transpose_v_joint(qkv_i[:, 2 * W:], qkv_t[:, 2 * W:], heads, hd, seg_i, seg_t, seg_j)
    o_i, o_t = ops.joint_attention_q_prescaled(qkv_i[:, :W], qkv_t[:, :W], qkv_i[:, W:2 * W], qkv_t[:, W:2 * W],
                                               vt, seg_i, seg_t, seg_j, heads, hd)
    r_i, r_t = torch.zeros_like(o_i, dtype=torch.float32), torch.zeros_like(o_t, dtype=torch.float32)
    for m in range(len(li)):
        rows = torch.cat([qkv_i[cu_i[m]:cu_i[m + 1]], qkv_t[cu_t[m]:cu_t[m + 1]]]).float()
        if rows.shape[0] == 0:
            continue
        q = (rows[:, :W] / ops.LOG2E).view(-1, heads, hd).transpose(0, 1)
        k = rows[:, W:2 * W].view(-1, heads, hd).transpose(0, 1)
        v = rows[:, 2 * W:].view(-1, heads, hd).transpose(0, 1)
        o = torch.matmul(torch.softmax(torch.matmul(q, k.transpose(1, 2).contiguous()), dim=-1), v)
        o = o.transpose(0, 1).reshape(-1, W)
        r_i[cu_i[m]:cu_i[m + 1]], r_t[cu_t[m]:cu_t[m + 1]] = o[:li[m]], o[li[m]:]
    for got, ref, name in ((o_i, r_i, "image"), (o_t, r_t, "text")):
        cos, rel = _metrics(got.float(), ref)
        print(f"joint img{li} txt{lt} heads {heads} ({name} rows): cos {cos:.6f} rel {rel:.2e}")
        assert torch.isfinite(got.float()).all() and cos >= 0.9999 and rel <= 1e-2


ROW_RANDOM = []
for _ in range(16):
    ROW_RANDOM.append((RNG.randint(1, 3000), 8 * RNG.randint(1, 768), RNG.choice(["ln", "rms"]),
                       RNG.choice(["mod", "affine", "plain"])))


@pytest.mark.parametrize("T,D,kind,form", ROW_RANDOM)
def test_adaln_random_shapes(T, D, kind, form):
    ops = _ops()
    g = _g(T * 5 + D)
    x = (torch.randn((T, D), generator=g, device=DEV) * 3 + 1).bfloat16()
    kw, rng = {}, random.Random(T * 17 + D)
    norm = (lambda t: oc.layer_norm(t, 1e-6)) if kind == "ln" else (lambda t: oc.rms_norm(t, None, 1e-6))
    ref = norm(x.float())
    if form == "mod":
        nseg = rng.randint(1, 4) if T >= 4 else 1
        cuts = sorted(rng.sample(range(1, T), nseg - 1)) if nseg > 1 else []
        cu = [0, *cuts, T]
        mod = torch.randn((len(cu) - 1, 2 * D), generator=g, device=DEV) * 0.1
        shift, scale = mod[:, :D], mod[:, D:]
        kw.update(shift=shift, scale=scale, segments=ops.Segments(cu, DEV))
        sh = torch.cat([shift[i].expand(cu[i + 1] - cu[i], D) for i in range(len(cu) - 1)])
        sc = torch.cat([scale[i].expand(cu[i + 1] - cu[i], D) for i in range(len(cu) - 1)])
        ref = ref * (1.0 + sc) + sh
    elif form == "affine":
        wt = 1.0 + 0.1 * torch.randn((D,), generator=g, device=DEV)
        bs = 0.1 * torch.randn((D,), generator=g, device=DEV)
        kw.update(weight=wt, bias=bs)
        ref = ref * wt + bs
    out = ops.adaln(x, kind=kind, **kw).float()
    cos, rel = _metrics(out, ref)
    print(f"adaln {kind} {form} {T}x{D}: cos {cos:.7f} rel {rel:.2e}")
    assert torch.isfinite(out).all() and cos >= 0.99999 and rel <= 5e-3


QK_RANDOM = []
for _ in range(10):
    hd = RNG.choice([64, 128])
    QK_RANDOM.append((RNG.randint(1, 3000), hd, RNG.randint(1, 6144 // hd), RNG.random() < 0.5))


@pytest.mark.parametrize("T,hd,heads,per_head", QK_RANDOM)
def test_qk_norm_random_shapes(T, hd, heads, per_head):
    ops = _ops()
    D = heads * hd
    g = _g(T * 11 + D)
    qkv = (torch.randn((T, 3 * D), generator=g, device=DEV) * 2).bfloat16()
    q0, k0, v0 = qkv[:, :D].float(), qkv[:, D:2 * D].float(), qkv[:, 2 * D:].clone()
    n = hd if per_head else D
    wq = 1.0 + 0.1 * torch.randn((n,), generator=g, device=DEV)
    wk = 1.0 + 0.1 * torch.randn((n,), generator=g, device=DEV)
    wq_full, wk_full = (wq.repeat(heads), wk.repeat(heads)) if per_head else (wq, wk)
    ops.qk_norm_rope_(qkv[:, :D], qkv[:, D:2 * D], wq_full.contiguous(), wk_full.contiguous(), hd, 1e-6,
                      per_head=per_head)

    def ref(x, w):
        if per_head:
            return oc.rms_norm(x.view(T, heads, hd), w, 1e-6).reshape(T, D)
        return oc.rms_norm(x, w, 1e-6)
    for got, x, w, name in ((qkv[:, :D], q0, wq, "q"), (qkv[:, D:2 * D], k0, wk, "k")):
        cos, rel = _metrics(got.float(), ref(x, w))
        print(f"qk_norm {name} T={T} heads={heads} hd={hd} per_head={per_head}: cos {cos:.7f} rel {rel:.2e}")
        assert cos >= 0.99999 and rel <= 5e-3
    assert torch.equal(qkv[:, 2 * D:], v0)  # the V columns of the buffer are not touched

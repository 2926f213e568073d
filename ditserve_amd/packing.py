"""Host-side packed-batch bookkeeping (integer, bit-exact).

Same contracts as the reference's build_cu_seqlens / packing_stats /
_build_packed_batch_plan (workers/ditserve/models/sd35_batch.py:135-176,230-317):
token prefix sums, padding statistics and the joint image+text layout, where
each segment's image tokens are followed by its text tokens.
"""
import itertools


def build_cu_seqlens(lengths):
    """[0, L0, L0+L1, ...]; every length must be a positive integer."""
    lengths = [int(n) for n in lengths]
    if any(n <= 0 for n in lengths):
        raise ValueError("sequence length must be positive")
    return [0, *itertools.accumulate(lengths)]


def packing_stats(heights, widths, *, vae_scale_factor=8, patch_size=2):
    """Token counts, cu_seqlens and padding savings of a resolution batch."""
    if len(heights) != len(widths) or not heights:
        raise ValueError("heights and widths must be non-empty sequences of equal length")
    stride = max(1, int(vae_scale_factor) * int(patch_size))
    res = [(int(h), int(w)) for h, w in zip(heights, widths)]
    for h, w in res:
        if h <= 0 or w <= 0 or h % stride or w % stride:
            raise ValueError(f"resolution ({h}, {w}) must be positive and divisible by {stride}")
    counts = [(h // stride) * (w // stride) for h, w in res]
    return {
        "batch_size": len(counts),
        "heterogeneous_resolutions": len(set(res)) > 1,
        "resolutions": [list(r) for r in res],
        **token_packing_stats(counts),
    }


def token_packing_stats(counts):
    """cu_seqlens and padding savings of a packed batch of token counts."""
    counts = [int(n) for n in counts]
    cu = build_cu_seqlens(counts)
    padded = len(counts) * max(counts)
    saved = padded - cu[-1]
    return {
        "image_token_counts": counts,
        "cu_seqlens": cu,
        "max_seqlen": max(counts),
        "packed_image_tokens": cu[-1],
        "padded_image_tokens": padded,
        "padding_saved_tokens": saved,
        "padding_waste_ratio": round(saved / padded, 4) if padded else 0.0,
        "packing_efficiency": round(cu[-1] / padded, 4) if padded else 1.0,
    }


def joint_layout(img_counts, txt_counts):
    """Joint image+text layout of a packed MMDiT batch.

    Returns cu_img, cu_txt, cu_joint (cu_joint[m] = cu_img[m] + cu_txt[m]),
    max_seqlen_img, max_seqlen_joint and the joint row of every image / text
    token (img_in_joint, txt_in_joint)."""
    if len(img_counts) != len(txt_counts) or not img_counts:
        raise ValueError("image and text counts must be non-empty lists of equal length")
    cu_img = build_cu_seqlens(img_counts)
    cu_txt = [0, *itertools.accumulate(int(n) for n in txt_counts)]
    cu_joint = [a + b for a, b in zip(cu_img, cu_txt)]
    img_in_joint, txt_in_joint = [], []
    for m, (ni, nt) in enumerate(zip(img_counts, txt_counts)):
        img_in_joint.extend(range(cu_joint[m], cu_joint[m] + ni))
        txt_in_joint.extend(range(cu_joint[m] + ni, cu_joint[m + 1]))
    return {
        "cu_img": cu_img,
        "cu_txt": cu_txt,
        "cu_joint": cu_joint,
        "max_seqlen_img": max(img_counts),
        "max_seqlen_joint": max(a + b for a, b in zip(img_counts, txt_counts)),
        "total_joint": cu_joint[-1],
        "img_in_joint": img_in_joint,
        "txt_in_joint": txt_in_joint,
    }


def wan_grid(latent_shape, patch=(1, 2, 2)):
    """(F', H', W') token grid of a Wan latent [..., C, F, H, W]."""
    f, h, w = latent_shape[-3:]
    pt, ph, pw = patch
    if f % pt or h % ph or w % pw:
        raise ValueError(f"latent {tuple(latent_shape)} not divisible by patch {patch}")
    return (f // pt, h // ph, w // pw)

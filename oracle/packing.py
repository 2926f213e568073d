"""Oracle: cu_seqlens / segment bookkeeping for packed batches (integer, bit-exact).

Follows workers/ditserve/models/sd35_batch.py:135-176 (build_cu_seqlens,
packing_stats) and :230-317 (_build_packed_batch_plan).  Pure Python ints.
"""


def build_cu_seqlens(lengths):
    """sd35_batch.py:135-145 — prefix sums [0, L0, L0+L1, ...]; lengths must be > 0."""
    cu = [0]
    for n in lengths:
        n = int(n)
        if n <= 0:
            raise ValueError("sequence length must be positive")
        cu.append(cu[-1] + n)
    return cu


def packing_stats(heights, widths, vae_scale_factor=8, patch_size=2):
    """sd35_batch.py:148-176 — token counts and padding savings for a resolution batch."""
    if len(heights) != len(widths) or not heights:
        raise ValueError("heights and widths must be non-empty sequences of equal length")
    stride = max(1, int(vae_scale_factor) * int(patch_size))
    counts = []
    for h, w in zip(heights, widths):
        h, w = int(h), int(w)
        if h <= 0 or w <= 0 or h % stride or w % stride:
            raise ValueError(f"resolution ({h}, {w}) must be positive and divisible by {stride}")
        counts.append((h // stride) * (w // stride))
    cu = build_cu_seqlens(counts)
    packed = cu[-1]
    padded = len(counts) * max(counts)
    saved = padded - packed
    return {
        "batch_size": len(counts),
        "heterogeneous_resolutions": len(set(zip(heights, widths))) > 1,
        "resolutions": [[int(h), int(w)] for h, w in zip(heights, widths)],
        "image_token_counts": counts,
        "cu_seqlens": cu,
        "max_seqlen": max(counts),
        "packed_image_tokens": packed,
        "padded_image_tokens": padded,
        "padding_saved_tokens": saved,
        "padding_waste_ratio": round(saved / padded, 4) if padded > 0 else 0.0,
        "packing_efficiency": round(packed / padded, 4) if padded > 0 else 1.0,
    }


def packed_plan(img_counts, txt_counts):
    """sd35_batch.py:230-317 — joint layout: per segment, image tokens then text tokens.

    Returns dict with cu_img, cu_txt, cu_joint, img_seg_ids, txt_seg_ids,
    img_in_joint_idx, txt_in_joint_idx, max_seqlen_img, max_seqlen_joint.
    """
    cu_img = build_cu_seqlens(img_counts)
    cu_txt = build_cu_seqlens(txt_counts)
    m = len(img_counts)
    cu_joint = [cu_img[i] + cu_txt[i] for i in range(m + 1)]
    img_seg = [s for s, n in enumerate(img_counts) for _ in range(n)]
    txt_seg = [s for s, n in enumerate(txt_counts) for _ in range(n)]
    img_idx = [j for s in range(m) for j in range(cu_joint[s], cu_joint[s] + img_counts[s])]
    txt_idx = [j for s in range(m) for j in range(cu_joint[s] + img_counts[s], cu_joint[s + 1])]
    return {
        "cu_img": cu_img,
        "cu_txt": cu_txt,
        "cu_joint": cu_joint,
        "img_seg_ids": img_seg,
        "txt_seg_ids": txt_seg,
        "img_in_joint_idx": img_idx,
        "txt_in_joint_idx": txt_idx,
        "max_seqlen_img": max(img_counts),
        "max_seqlen_joint": max(a + b for a, b in zip(img_counts, txt_counts)),
        "total_joint": cu_joint[-1],
    }


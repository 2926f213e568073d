"""cu_seqlens / packing bookkeeping: oracle and product against the reference's golden vectors."""
import json
import os

import pytest

from ditserve_amd import packing
from oracle import packing as opack

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "packing_vectors.json")))


@pytest.mark.parametrize("impl", [opack, packing], ids=["oracle", "product"])
def test_ragged_packing_stats(impl):
    g = GOLD["ragged"]
    st = impl.packing_stats(g["heights"], g["widths"], vae_scale_factor=g["vae_scale_factor"],
                            patch_size=g["patch_size"])
    for key in ("image_token_counts", "cu_seqlens", "packed_image_tokens", "max_seqlen",
                "padded_image_tokens", "padding_saved_tokens", "padding_waste_ratio"):
        assert st[key] == g[key], key
    assert st["heterogeneous_resolutions"] is True
    assert impl.build_cu_seqlens(g["image_token_counts"]) == g["cu_seqlens"]


@pytest.mark.parametrize("impl", [opack, packing], ids=["oracle", "product"])
def test_build_cu_seqlens_rejects_nonpositive(impl):
    with pytest.raises(ValueError):
        impl.build_cu_seqlens([3, 0, 2])
    with pytest.raises(ValueError):
        impl.packing_stats([512], [500])


@pytest.mark.parametrize("impl", [opack, packing], ids=["oracle", "product"])
def test_toy_and_dispatch_vectors(impl):
    g = GOLD["toy_cu_seqlens_img"]
    assert impl.build_cu_seqlens(g["counts"]) == g["cu"]
    d = GOLD["varlen_dispatch"]
    plan = opack.packed_plan(d["img_counts"], d["txt_counts"]) if impl is opack else \
        packing.joint_layout(d["img_counts"], d["txt_counts"])
    assert plan["cu_joint"] == d["joint_call"]["cu"]
    assert plan["max_seqlen_joint"] == d["joint_call"]["max"]
    assert plan["total_joint"] == d["joint_call"]["q_shape_rows"]
    assert plan["cu_img"] == d["image_only_call"]["cu"]
    assert plan["max_seqlen_img"] == d["image_only_call"]["max"]


def test_joint_index_maps_agree():
    for img, txt in ([[4, 9], [3, 3]], [[4096, 1024, 7], [333, 333, 1]], [[1], [5]]):
        o = opack.packed_plan(img, txt)
        p = packing.joint_layout(img, txt)
        assert o["img_in_joint_idx"] == p["img_in_joint"]
        assert o["txt_in_joint_idx"] == p["txt_in_joint"]
        assert o["cu_joint"] == p["cu_joint"]
        # the two maps partition the joint rows
        assert sorted(p["img_in_joint"] + p["txt_in_joint"]) == list(range(p["total_joint"]))


def test_build_config_vectors():
    w = GOLD["wan_packed"]
    counts = [f * h * ww for f, h, ww in w["grids"]]
    assert packing.build_cu_seqlens(counts) == w["cu_q"] == opack.build_cu_seqlens(counts)
    assert packing.build_cu_seqlens([512] * 4) == w["cu_k_text"]
    s = GOLD["sd35_packed"]
    lay = packing.joint_layout(s["img_counts"], s["txt_counts"])
    assert lay["cu_img"] == s["cu_img"] and lay["cu_joint"] == s["cu_joint"]
    assert packing.wan_grid((16, 21, 60, 104)) == (21, 30, 52)

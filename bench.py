#!/usr/bin/env python3
"""Benchmark: one Wan2.1-T2V-1.3B denoise step at 480x832x81 frames with CFG batch 2
(2 x 32760 tokens), bf16, on one MI355X -- plus the other single-GPU workloads of
the same path, each measured in the same run and reported under ``per_config``.

Headline step = packed prelude for the (cond, uncond) pair + 30 DiT blocks +
prediction + the fused CFG combine and UniPC update (Wan's scheduler recipe: flow
sigmas, shift 3.0, 50-step schedule, order 2 with corrector), all on the ditk HIP
kernels.  The model timestep of each step is the schedule's (999, 997, ...).
Synthetic data: random-init weights N(0, 0.02^2) (norm weights N(1, 0.02^2)),
latent 16x21x60x104 N(0,1), text contexts 512x4096 N(0,1) with 120 (cond) and 0
(uncond) valid rows.

``per_config`` adds, each with its own steps/s (or forwards/s), tokens/s,
attention roofline fraction and CPU baseline:
  * wan21_block_1560tok   one Wan2.1 block, 1x30x52 grid (1560 tokens), 77 valid
                          text rows, t = 500 (GPU bf16 vs the oracle in fp32 on CPU);
  * wan21_packed_4req     four requests packed into one varlen batch (grids 21x30x52,
                          9x30x52, 13x20x32, 5x16x16 = 56400 tokens), own timesteps
                          U[0,1000) and texts (valid 30-200): one packed forward;
  * sd35_medium_1024_cfg2 SD3.5-Medium 1024^2 step, CFG pair of joint segments
                          (4096 image + 333 text tokens each), FlowMatch-Euler;
  * sd35_packed_2x1024_4x512_cfg2  SD3.5-Medium packed step over 2 x 1024^2 +
                          4 x 512^2 requests, each a CFG pair (12 joint segments),
                          per-request FlowMatch-Euler;
  * wan22_ti2v_5b_704p_cfg2  Wan2.2-TI2V-5B 704x1280x121f step, CFG pair of
                          2 x 27280 tokens, text valid 150/0, t = 700 schedule;
  * wan21_720p_cfg2       Wan2.1-T2V-1.3B 720x1280x81f step, CFG pair of 2 x 75600
                          tokens (latent 16x21x90x160), UniPC flow shift 5;
  * wan21_480p_33f_cfg2   Wan2.1-T2V-1.3B 480x832x33f step (the reference's dev
                          shape), CFG pair of 2 x 14040 tokens.

Prints one JSON line.  ``roofline`` is for the dominant kernel, the self-attention
flash kernel, from HIP events recorded on its launch stream over the timed steps.
``kernels`` (per config) gives every hot kernel's roofline -- GEMMs and attention
as TFLOP/s of the 2.5 PFLOP/s bf16 peak, the row kernels as TB/s of 8 TB/s HBM --
from HIP events around each kernel over one more step after the timed ones.
``cpu_baseline`` times the oracle (the CPU fp32 restatement of the reference block)
on one full-shape block-forward and extrapolates to the step (blocks x branches).
"""
import argparse
import json
import math
import os
import sys
import time

PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_TBS = 8.0
CALIB_BYTES = 256 << 20
GUIDANCE = 5.0
SCHEDULE_STEPS = 50
# HBM traffic of one headline self-attention launch, from two rocprofv3 --pmc passes
# over this bench (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by that
# counter's reading for the CALIB_BYTES copy: FETCH 884805 KiB x 1.9998, WRITE
# 196560 KiB x 1.0000 (profiles/wan21_480p_cfg2_step_traffic.md).
ATTN_SELF_TRAFFIC_BYTES = (884805 * 1.9998 + 196560 * 1.0000) * 1024

WAN21_METRIC = "denoise steps/s & tokens/s, Wan2.1-1.3B 480p-81f CFG2; attn % bf16 MFMA peak"
WORKLOADS = {
    "wan21_480p": dict(
        metric=WAN21_METRIC, arch="wan21", latent=(16, 21, 60, 104), text_valid=(120, 0), flow_shift=3.0,
        ref_ms=3964.62),
    "wan21_480p_33f": dict(
        metric="denoise steps/s & tokens/s, Wan2.1-1.3B 480p-33f CFG2; attn % bf16 MFMA peak",
        arch="wan21", latent=(16, 9, 60, 104), text_valid=(120, 0), flow_shift=3.0, ref_ms=1149.62),
    "wan21_720p": dict(
        metric="denoise steps/s & tokens/s, Wan2.1-1.3B 720p-81f CFG2; attn % bf16 MFMA peak",
        arch="wan21", latent=(16, 21, 90, 160), text_valid=(120, 0), flow_shift=5.0, ref_ms=16212.46),
    "wan22_ti2v_5b_704p": dict(
        metric="denoise steps/s & tokens/s, Wan2.2-TI2V-5B 704p-121f CFG2; attn % bf16 MFMA peak",
        arch="wan22", latent=(48, 31, 44, 80), text_valid=(150, 0), flow_shift=5.0, ref_ms=7813.18),
    "sd35_medium_1024": dict(
        metric="denoise steps/s & tokens/s, SD3.5-Medium 1024x1024 CFG2; joint attn % bf16 MFMA peak",
        latent=(16, 128, 128), text_len=333, steps=28, shift=3.0, ref_ms=217.23),
    "sd35_packed_2x1024_4x512": dict(
        metric="packed denoise steps/s & tokens/s, SD3.5-Medium 2x1024^2 + 4x512^2 requests, CFG2 each "
               "(12 joint segments); joint attn % bf16 MFMA peak",
        sizes=(1024, 1024, 512, 512, 512, 512), text_len=333, steps=28, shift=3.0, guidance=7.0),
    "wan21_packed_4req": dict(
        metric="packed forwards/s & tokens/s, Wan2.1-1.3B 4-request varlen batch (56400 tokens); "
               "attn % bf16 MFMA peak",
        shapes=[(16, 21, 60, 104), (16, 9, 60, 104), (16, 13, 40, 64), (16, 5, 32, 32)]),
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-per-config", action="store_true", help="headline workload only")
    ap.add_argument("--breakdown", action="store_true", help="per-op HIP-event breakdown in the JSON")
    ap.add_argument("--surfaces", action="store_true",
                    help="only time the reference-shaped entry points against the engine path (one JSON line)")
    ap.add_argument("--workload", default="wan21_480p", choices=sorted(WORKLOADS),
                    help="the workload of the top-level line (default: the Wan2.1 480p headline)")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# CPU baselines: the oracle (CPU fp32 restatement of the reference arithmetic)
# ---------------------------------------------------------------------------

def cpu_threads():
    """Threads for the CPU baseline: the host's cores, bounded by the CPUs this
    process may run on and by OMP_NUM_THREADS when the environment sets it."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return n


def _cpu_info(threads, kind="port"):
    return {"cores": threads, "threads": threads, "host_cores": os.cpu_count(), "kind": kind}


def cpu_wan_block_s(cfg, seqs, text_len=512, seed=0):
    """Seconds for one oracle Wan block-forward over `seqs` (a packed batch when
    several), fp32, torch's CPU flash SDPA.  A warm-up on a small slice first."""
    import torch

    from ditserve_amd.wan import WanConfig, random_state_dict
    from oracle import common as oc
    from oracle import wan as ow

    one = WanConfig(**{**cfg.as_dict(), "layers": 1})
    sd = random_state_dict(one, seed=seed)
    g = torch.Generator().manual_seed(seed + 2)
    grids = [s for s in seqs]
    counts = [f * h * w for f, h, w in grids]
    h = torch.randn(sum(counts), cfg.dim, generator=g)
    encs = [torch.randn(text_len, cfg.dim, generator=g) for _ in counts]
    projs = torch.randn(len(counts), 6, cfg.dim, generator=g) * 0.02
    rot = [ow.rope_freqs(gr, cfg.head_dim) for gr in grids]
    w = min(counts[0], 1560)
    ow.block_forward(sd, 0, h[:w], encs[0], projs[0], rot[0][0][:w], rot[0][1][:w], cfg.heads, attn=oc.sdpa_fast)
    cu = [0]
    for n in counts:
        cu.append(cu[-1] + n)
    t0 = time.perf_counter()
    ow.block_forward_packed(sd, 0, h, cu, encs, projs, rot, cfg.heads, attn=oc.sdpa_fast)
    return time.perf_counter() - t0


def cpu_baseline_wan_step(cfg, grid, threads, label):
    """configs with a CFG pair: one block-forward at the full shape (one branch),
    extrapolated x (layers x 2 branches)."""
    s = cpu_wan_block_s(cfg, [grid])
    seq = grid[0] * grid[1] * grid[2]
    step_s = s * cfg.layers * 2
    return dict(value=1.0 / step_s, unit="steps/s", tokens_per_s=2 * seq / step_s, block_s=s,
                sample=f"1 {label} block-forward at S={seq} (one CFG branch), fp32, CPU flash SDPA, {threads} "
                       f"threads: {s:.2f} s; extrapolated x{cfg.layers * 2} ({cfg.layers} blocks x 2 branches)",
                **_cpu_info(threads))


def cpu_baseline_wan_packed(cfg, grids, threads):
    s = cpu_wan_block_s(cfg, grids)
    tokens = sum(f * h * w for f, h, w in grids)
    fwd_s = s * cfg.layers
    return dict(value=1.0 / fwd_s, unit="forwards/s", tokens_per_s=tokens / fwd_s, block_s=s,
                sample=f"1 Wan2.1 block-forward over the 4-request packed batch ({tokens} tokens, per-segment CPU "
                       f"flash SDPA), fp32, {threads} threads: {s:.2f} s; extrapolated x{cfg.layers} blocks",
                **_cpu_info(threads))


def cpu_baseline_wan_block(cfg, threads, repeats=5):
    """One Wan2.1 block on the 1x30x52 grid: 2 warm-ups, median of `repeats`."""
    import torch

    from ditserve_amd.wan import WanConfig, random_state_dict
    from oracle import wan as ow

    one = WanConfig(**{**cfg.as_dict(), "layers": 1})
    sd = random_state_dict(one, seed=0)
    g = torch.Generator().manual_seed(2)
    h = torch.randn(1560, cfg.dim, generator=g)
    enc = torch.randn(512, cfg.dim, generator=g)
    enc[77:] = 0
    proj = torch.randn(6, cfg.dim, generator=g) * 0.02
    cos, sin = ow.rope_freqs((1, 30, 52))
    times = []
    for i in range(2 + repeats):
        t0 = time.perf_counter()
        ow.block_forward(sd, 0, h, enc, proj, cos, sin, cfg.heads)
        if i >= 2:
            times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    return dict(value=1000.0 * med, unit="ms/block", block_s=med,
                sample=f"Wan2.1 block, 1560 tokens, 512 text rows, fp32 (oracle's exact SDPA), {threads} threads: "
                       f"median of {repeats} after 2 warm-ups", **_cpu_info(threads))


def _cpu_sd35_block_s(cfg, n_img, text_len):
    """Seconds of one dual-attention and one plain oracle SD3.5 joint block on one
    segment (n_img image + text_len text tokens), fp32, torch's CPU flash SDPA."""
    import torch

    from ditserve_amd.sd35 import SD35Config, random_state_dict
    from oracle import common as oc
    from oracle import sd35 as osd

    two = SD35Config(**{**cfg.__dict__, "layers": 3, "dual_layers": (0,)})
    sd = random_state_dict(two, seed=0)
    g = torch.Generator().manual_seed(3)
    h = torch.randn(n_img, cfg.dim, generator=g)
    c = torch.randn(text_len, cfg.dim, generator=g)
    temb = torch.randn(cfg.dim, generator=g)
    ocfg = dict(heads=cfg.heads, eps=cfg.eps, layers=3, dual_layers=(0,))
    osd.joint_block(sd, 1, h[:256], c[:32], temb, ocfg, attn=oc.sdpa_fast)  # warm-up
    times = {}
    for name, i in (("dual", 0), ("plain", 1)):
        t0 = time.perf_counter()
        osd.joint_block(sd, i, h, c, temb, ocfg, attn=oc.sdpa_fast)
        times[name] = time.perf_counter() - t0
    return times["dual"], times["plain"]


def cpu_baseline_sd35(cfg, n_img, text_len, threads):
    """One dual-attention and one plain SD3.5 joint block on one CFG branch
    (n_img image + text_len text tokens), extrapolated to the step:
    2 branches x (dual x 13 + plain x 11) -- the last block, which drops its
    text stream, is counted as plain."""
    dual, plain = _cpu_sd35_block_s(cfg, n_img, text_len)
    n_dual = len(cfg.dual_layers)
    step_s = 2 * (dual * n_dual + plain * (cfg.layers - n_dual))
    return dict(value=1.0 / step_s, unit="steps/s", tokens_per_s=2 * n_img / step_s, dual_block_s=dual,
                plain_block_s=plain,
                sample=f"1 dual + 1 plain SD3.5-M joint block ({n_img} image + {text_len} text tokens, one CFG "
                       f"branch), fp32, CPU flash SDPA, {threads} threads: {dual:.2f} s + "
                       f"{plain:.2f} s; extrapolated x2 branches x ({n_dual} dual + "
                       f"{cfg.layers - n_dual} plain blocks)", **_cpu_info(threads))


def cpu_baseline_sd35_packed(cfg, sizes, text_len, threads):
    """The packed batch's blocks are per-segment on the CPU: one dual and one plain
    joint block per distinct request size (one CFG branch), extrapolated to the
    step as sum over requests of 2 branches x (dual x 13 + plain x 11)."""
    per = {size: _cpu_sd35_block_s(cfg, (size // 16) ** 2, text_len) for size in sorted(set(sizes))}
    n_dual = len(cfg.dual_layers)
    step_s = sum(2 * (per[s][0] * n_dual + per[s][1] * (cfg.layers - n_dual)) for s in sizes)
    n_img = sum(2 * (s // 16) ** 2 for s in sizes)
    parts = ", ".join(f"{s}^2 ({(s // 16) ** 2} image tokens): {per[s][0]:.2f} s + {per[s][1]:.2f} s"
                      for s in sorted(per))
    return dict(value=1.0 / step_s, unit="steps/s", tokens_per_s=n_img / step_s,
                block_s={str(s): {"dual": per[s][0], "plain": per[s][1]} for s in per},
                sample=f"1 dual + 1 plain SD3.5-M joint block per request size, one segment with {text_len} text "
                       f"tokens, fp32, CPU flash SDPA, {threads} threads: {parts}; extrapolated over the 6 requests "
                       f"x 2 branches x ({n_dual} dual + {cfg.layers - n_dual} plain blocks)", **_cpu_info(threads))


# ---------------------------------------------------------------------------
# GPU workloads
# ---------------------------------------------------------------------------

def _roofline(kernel, flops_per_launch, region, traffic=None, algorithmic_bytes=None):
    tflops = flops_per_launch / (region["avg_ms"] * 1e-3) / 1e12
    out = {"kernel": kernel, "bound": "mfma", "achieved": tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
           "frac": tflops / PEAK_BF16_TFLOPS, "traffic": traffic, "avg_launch_ms": region["avg_ms"],
           "launches": region["count"], "flops_per_launch": flops_per_launch}
    if traffic is not None:
        out["traffic_unit"] = "bytes/launch"
    if algorithmic_bytes is not None:
        out["algorithmic_bytes"] = algorithmic_bytes
    return out


KERNEL_STEPS = 1


def _timed(step, state, steps, warmup, prof_model, only, breakdown):
    """Run warmup + timed steps; returns (state, ms per step, region summary of the
    timed steps, region summary of every region over KERNEL_STEPS further steps).

    The timed steps record events only around the `only` regions (each event pair
    costs host time); the per-kernel table comes from the extra steps after the
    timed region, with every region recorded, and does not enter ms per step."""
    import torch

    from ditserve_amd.profiling import EventProfiler

    for _ in range(warmup):
        state = step(state)
    torch.cuda.synchronize()
    prof = EventProfiler(enabled=True, only=None if breakdown else only)
    prof_model.profiler = prof
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        state = step(state)
    end.record()
    torch.cuda.synchronize()
    kprof = EventProfiler(enabled=True)
    prof_model.profiler = kprof
    for _ in range(KERNEL_STEPS):
        state = step(state)
    torch.cuda.synchronize()
    prof_model.profiler = EventProfiler(enabled=False)
    return state, start.elapsed_time(end) / steps, prof.summary(), kprof.summary()


def _kernel_table(regions, spec):
    """{name: roofline entry} from HIP-event region averages.  spec: {region: (bound,
    work per region occurrence, what the region holds)}; "mfma" work is FLOP, "hbm"
    work is algorithmic bytes (minimal reads + writes)."""
    out = {}
    for name, (bound, work, what) in spec.items():
        r = regions.get(name)
        if not r:
            continue
        sec = r["avg_ms"] * 1e-3
        if bound == "mfma":
            ach, peak, unit = work / sec / 1e12, PEAK_BF16_TFLOPS, "TFLOP/s"
        else:
            ach, peak, unit = work / sec / 1e12, PEAK_HBM_TBS, "TB/s"
        out[name] = {"what": what, "bound": bound, "achieved": ach, "peak": peak, "unit": unit,
                     "frac": ach / peak, "avg_launch_ms": r["avg_ms"], "launches": r["count"],
                     ("flops_per_launch" if bound == "mfma" else "bytes_per_launch"): work}
    return out


def _wan_kernel_spec(cfg, seqs, text_len):
    """Per-kernel work of one Wan block over the packed rows (M = all tokens)."""
    M, D, F = sum(seqs), cfg.dim, cfg.ffn
    return {
        "attn_self": ("mfma", 4.0 * sum(s * s for s in seqs) * D, "self-attention flash kernel"),
        "attn_cross": ("mfma", 4.0 * M * text_len * D, f"cross-attention over {text_len} text keys per segment"),
        "gemm_qkv": ("mfma", 2.0 * M * 3 * D * D, f"fused QKV projection {M}x{3 * D}x{D}, bias"),
        "gemm_o_gate": ("mfma", 2.0 * M * D * D, f"self-attention output projection {M}x{D}x{D}, gated residual"),
        "gemm_cross_q": ("mfma", 2.0 * M * D * D, f"cross-attention q projection {M}x{D}x{D}, bias"),
        "gemm_o_res": ("mfma", 2.0 * M * D * D, f"cross-attention output projection {M}x{D}x{D}, residual"),
        "gemm_ffn_up_gelu": ("mfma", 2.0 * M * F * D, f"FFN up {M}x{F}x{D}, GELU-tanh"),
        "gemm_ffn_down_gate": ("mfma", 2.0 * M * D * F, f"FFN down {M}x{D}x{F}, gated residual"),
        "adaln": ("hbm", 4.0 * M * D, "AdaLN (LayerNorm + per-segment shift/scale), bf16 in + out"),
        "qk_norm_rope": ("hbm", 8.0 * M * D, "QK RMSNorm across heads + 3D RoPE, in place on q and k"),
        "transpose_v": ("hbm", 4.0 * M * D, "V -> per-head transposed Vt staging, bf16 in + out"),
    }


def _sd35_kernel_spec(cfg, img_counts, txt_counts):
    """Per-kernel work of one SD3.5 joint block over the packed rows."""
    D, F = cfg.dim, cfg.ffn
    Mi, Mt = sum(img_counts), sum(txt_counts)
    joint = sum((n + l) ** 2 for n, l in zip(img_counts, txt_counts))
    return {
        "attn_joint": ("mfma", 4.0 * joint * D, "joint image+text attention, head_dim 64"),
        "attn_dual_core": ("mfma", 4.0 * sum(n * n for n in img_counts) * D, "dual image-only attention, head_dim 64"),
        "gemm_qkv_img": ("mfma", 2.0 * Mi * 3 * D * D, f"image QKV {Mi}x{3 * D}x{D}, bias"),
        "gemm_qkv_txt": ("mfma", 2.0 * Mt * 3 * D * D, f"text QKV {Mt}x{3 * D}x{D}, bias"),
        "gemm_out_pair": ("mfma", 2.0 * (Mi + Mt) * D * D,
                          f"image + text output projections ({Mi} + {Mt})x{D}x{D}, gated residual, one pair call"),
        "gemm_ffn_up_img": ("mfma", 2.0 * Mi * F * D, f"image FFN up {Mi}x{F}x{D}, GELU-tanh"),
        "gemm_ffn_down_pair": ("mfma", 2.0 * (Mi + Mt) * D * F,
                               f"image + text FFN down ({Mi} + {Mt})x{D}x{F}, gated residual, one pair call"),
        "qk_norm": ("hbm", 8.0 * (Mi + Mt) * D, "image and text per-head QK RMSNorm, in place on q and k, one launch"),
        "transpose_v_joint": ("hbm", 4.0 * (Mi + Mt) * D, "image + text V -> joint transposed Vt staging"),
    }


def _release():
    """Return the previous workload's device memory before the next one starts."""
    import gc

    import torch
    gc.collect()
    torch.cuda.empty_cache()


def calibration_copy():
    """The known-size copy (CALIB_BYTES read and written, outside any timing) that
    the HBM-traffic counters of a profile of this script are scaled by."""
    import torch
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
    torch.empty_like(src).copy_(src)
    torch.cuda.synchronize()


def run_wan_cfg(name, steps, warmup, breakdown=False):
    """Wan CFG-pair denoise step (Wan2.1 480p or Wan2.2-5B 704p)."""
    import torch

    from ditserve_amd.solver import UniPCFlowScheduler
    from ditserve_amd.wan import WAN21_T2V_1_3B, WAN22_TI2V_5B, WanTransformer, step_flops

    wl = WORKLOADS[name]
    cfg = WAN21_T2V_1_3B if wl["arch"] == "wan21" else WAN22_TI2V_5B
    latent_shape = wl["latent"]
    dev = "cuda"
    model = WanTransformer.random(cfg, seed=0, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    latent = torch.randn(latent_shape, generator=g, device=dev)
    texts = []
    for valid in wl["text_valid"]:
        t = torch.randn((cfg.text_len, cfg.text_dim), generator=g, device=dev)
        t[valid:] = 0
        texts.append(t)
    pt, ph, pw = cfg.patch
    grid = (latent_shape[1] // pt, latent_shape[2] // ph, latent_shape[3] // pw)
    seq = grid[0] * grid[1] * grid[2]
    sched = UniPCFlowScheduler(flow_shift=wl["flow_shift"])
    sched.set_timesteps(max(SCHEDULE_STEPS, warmup + steps + KERNEL_STEPS))

    def step(lat):
        t = float(sched.timesteps[sched.step_index])
        cond, uncond = model.forward_packed([lat, lat], [t, t], texts)
        return sched.step(cond, t, lat, uncond=uncond, guidance=GUIDANCE)[0]

    latent, ms, regions, kregions = _timed(step, latent, steps, warmup, model, {"attn_self"}, breakdown)
    if not bool(torch.isfinite(latent).all()):
        raise RuntimeError(f"{name}: non-finite latent after the timed steps")
    attn_flops = 4.0 * 2 * seq * seq * cfg.dim  # per launch: 2 segments (CFG pair), non-causal
    total_flops = step_flops(cfg, [seq, seq], cfg.text_len)
    arch = "Wan2.1-T2V-1.3B" if wl["arch"] == "wan21" else "Wan2.2-TI2V-5B"
    vae = 8 if wl["arch"] == "wan21" else 16  # the VAE's spatial stride; 4 frames per latent frame
    frames = f"{latent_shape[2] * vae}x{latent_shape[3] * vae}x{(latent_shape[1] - 1) * 4 + 1}f"
    out = {
        "metric": wl["metric"], "value": 1000.0 / ms, "unit": "steps/s", "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "tokens_per_s": 2 * seq * 1000.0 / ms,
        "workload": (f"{arch}-architecture denoise step, latent {'x'.join(map(str, latent_shape))} ({frames}), "
                     f"CFG pair packed as 2 x {seq} tokens, {cfg.layers} blocks, text 512 (valid "
                     f"{wl['text_valid'][0]}/{wl['text_valid'][1]}), UniPC flow-shift-{wl['flow_shift']:g} "
                     f"{SCHEDULE_STEPS}-step schedule"),
        "tokens_per_step": 2 * seq, "blocks": cfg.layers,
        "model_tflops": total_flops / (ms * 1e-3) / 1e12,
        "model_mfma_frac": total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": _roofline(f"flash_fwd_asm<128, true> (self-attention, 2 x {seq} tokens x {cfg.heads} heads)",
                              attn_flops, regions["attn_self"],
                              ATTN_SELF_TRAFFIC_BYTES if name == "wan21_480p" else None,
                              4.0 * 2 * seq * cfg.dim * 2),
        "kernels": _kernel_table(kregions, _wan_kernel_spec(cfg, [seq, seq], cfg.text_len)),
        "reference_a100_ms_per_step": wl["ref_ms"], "vs_reference_a100": wl["ref_ms"] / ms,
        "_grid": grid, "_cfg": cfg,
    }
    if breakdown:
        out["breakdown_ms_per_step"] = {k: v["total_ms"] / steps for k, v in regions.items()}
    return out


def run_wan_packed(steps, warmup, breakdown=False):
    """Four Wan2.1 requests packed into one varlen batch: one packed forward
    (prelude, 30 blocks, prediction) per step."""
    import torch

    from ditserve_amd.wan import WAN21_T2V_1_3B, WanTransformer, step_flops

    wl = WORKLOADS["wan21_packed_4req"]
    cfg, dev = WAN21_T2V_1_3B, "cuda"
    model = WanTransformer.random(cfg, seed=4, device=dev)
    g = torch.Generator().manual_seed(5)
    lats = [torch.randn(s, generator=g).to(dev) for s in wl["shapes"]]
    ts = [float(x) for x in (torch.rand(4, generator=g) * 1000)]
    valid = [int(x) for x in torch.randint(30, 201, (4,), generator=g)]
    texts = []
    for i in range(4):
        t = torch.randn((cfg.text_len, cfg.text_dim), generator=g)
        t[valid[i]:] = 0
        texts.append(t.to(dev))
    grids = [(s[1], s[2] // 2, s[3] // 2) for s in wl["shapes"]]
    seqs = [f * h * w for f, h, w in grids]

    def step(_):
        return model.forward_packed(lats, ts, texts)

    outs, ms, regions, kregions = _timed(step, None, steps, warmup, model, {"attn_self"}, breakdown)
    if not all(bool(torch.isfinite(o).all()) for o in outs):
        raise RuntimeError("packed Wan forward produced non-finite values")
    attn_flops = 4.0 * sum(s * s for s in seqs) * cfg.dim
    total_flops = step_flops(cfg, seqs, cfg.text_len)
    tokens = sum(seqs)
    out = {
        "metric": wl["metric"], "value": 1000.0 / ms, "unit": "forwards/s", "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "tokens_per_s": tokens * 1000.0 / ms,
        "workload": (f"Wan2.1-T2V-1.3B-architecture packed forward of 4 requests (grids "
                     f"{', '.join('x'.join(map(str, gr)) for gr in grids)} = {tokens} tokens, cu_seqlens "
                     f"[0, {', '.join(str(sum(seqs[:i + 1])) for i in range(4))}]), own timesteps U[0,1000) and "
                     f"512-row texts (valid {valid}), {cfg.layers} blocks, one branch each"),
        "tokens_per_step": tokens, "blocks": cfg.layers,
        "model_tflops": total_flops / (ms * 1e-3) / 1e12,
        "model_mfma_frac": total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": _roofline(f"flash_fwd_asm<128, true> (self-attention, 4 segments, {tokens} tokens x "
                              f"{cfg.heads} heads)", attn_flops, regions["attn_self"],
                              algorithmic_bytes=4.0 * tokens * cfg.dim * 2),
        "kernels": _kernel_table(kregions, _wan_kernel_spec(cfg, seqs, cfg.text_len)),
        "reference_a100_ms_per_step": None, "vs_reference_a100": None,
        "_grids": grids,
    }
    if breakdown:
        out["breakdown_ms_per_step"] = {k: v["total_ms"] / steps for k, v in regions.items()}
    return out


def run_sd35(steps, warmup, breakdown=False):
    """SD3.5-Medium 1024^2 denoise step, CFG as a packed pair of joint segments
    (4096 image + 333 text tokens each), 24 blocks, FlowMatch-Euler."""
    import torch

    from ditserve_amd.sd35 import SD35_MEDIUM, SD35Transformer, forward_packed_sd35, step_flops
    from ditserve_amd.solver import FlowMatchEulerScheduler

    wl = WORKLOADS["sd35_medium_1024"]
    cfg, dev = SD35_MEDIUM, "cuda"
    model = SD35Transformer.random(cfg, seed=0, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    latent = torch.randn(wl["latent"], generator=g, device=dev)
    text_c = torch.randn((wl["text_len"], cfg.text_dim), generator=g, device=dev)
    pooled_c = torch.randn((cfg.pooled_dim,), generator=g, device=dev)
    text_u, pooled_u = torch.zeros_like(text_c), torch.zeros_like(pooled_c)
    sched = FlowMatchEulerScheduler(shift=wl["shift"])
    sched.set_timesteps(max(wl["steps"], warmup + steps + KERNEL_STEPS))
    n_img = (wl["latent"][1] // cfg.patch) * (wl["latent"][2] // cfg.patch)
    n_joint = n_img + wl["text_len"]

    def step(lat):
        t = float(sched.timesteps[sched.step_index])
        outs, _ = forward_packed_sd35(torch, model, [lat.unsqueeze(0)] * 2, [t, t],
                                      [text_u.unsqueeze(0), text_c.unsqueeze(0)], [pooled_u, pooled_c])
        return sched.step(outs[1], t, lat, uncond=outs[0], guidance=7.0)[0]

    latent, ms, regions, kregions = _timed(step, latent, steps, warmup, model, {"attn_joint"}, breakdown)
    if not bool(torch.isfinite(latent).all()):
        raise RuntimeError("sd35: non-finite latent after the timed steps")
    attn_flops = 4.0 * 2 * n_joint * n_joint * cfg.dim
    total_flops = step_flops(cfg, [n_img, n_img], [wl["text_len"]] * 2)
    out = {
        "metric": wl["metric"], "value": 1000.0 / ms, "unit": "steps/s", "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "tokens_per_s": 2 * n_img * 1000.0 / ms,
        "workload": (f"SD3.5-Medium-architecture denoise step at 1024x1024 (latent 16x128x128), CFG pair packed "
                     f"as 2 x ({n_img} image + {wl['text_len']} text) joint tokens, {cfg.layers} blocks (13 with "
                     f"dual attention), FlowMatch-Euler shift {wl['shift']:g}"),
        "tokens_per_step": 2 * n_joint, "blocks": cfg.layers,
        "model_tflops": total_flops / (ms * 1e-3) / 1e12,
        "model_mfma_frac": total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": _roofline(f"flash_fwd_asm<64, true, true> (joint attention, 2 x {n_joint} tokens x {cfg.heads} heads)",
                              attn_flops, regions["attn_joint"], algorithmic_bytes=4.0 * 2 * n_joint * cfg.dim * 2),
        "kernels": _kernel_table(kregions, _sd35_kernel_spec(cfg, [n_img, n_img], [wl["text_len"]] * 2)),
        "reference_a100_ms_per_step": wl["ref_ms"], "vs_reference_a100": wl["ref_ms"] / ms,
        "_n_img": n_img, "_cfg": cfg,
    }
    if breakdown:
        out["breakdown_ms_per_step"] = {k: v["total_ms"] / steps for k, v in regions.items()}
    return out


def run_sd35_packed(steps, warmup, breakdown=False):
    """SD3.5-Medium packed batch of 2 x 1024^2 + 4 x 512^2 requests, each a CFG pair
    (unconditional then conditional segment, workers/ditserve/models/sd35.py:919-930):
    12 joint segments in one packed forward per step, then each request's own
    FlowMatch-Euler update on its CFG-combined output (step_members_once, the
    reference's _step_members_once)."""
    import torch

    from ditserve_amd.packing import build_cu_seqlens
    from ditserve_amd.sd35 import SD35_MEDIUM, SD35Transformer, step_flops, step_members_once
    from ditserve_amd.solver import FlowMatchEulerScheduler

    wl = WORKLOADS["sd35_packed_2x1024_4x512"]
    cfg, dev = SD35_MEDIUM, "cuda"
    model = SD35Transformer.random(cfg, seed=0, device=dev)
    g = torch.Generator(device=dev).manual_seed(7)
    n_steps = max(wl["steps"], warmup + steps + KERNEL_STEPS)
    states = []
    for size in wl["sizes"]:
        lat = torch.randn((1, 16, size // 8, size // 8), generator=g, device=dev)
        txt = torch.randn((1, wl["text_len"], cfg.text_dim), generator=g, device=dev)
        pooled = torch.randn((1, cfg.pooled_dim), generator=g, device=dev)
        sched = FlowMatchEulerScheduler(shift=wl["shift"])
        sched.set_timesteps(n_steps)
        emb = dict(prompt_embeds=txt, pooled_prompt_embeds=pooled, negative_prompt_embeds=torch.zeros_like(txt),
                   negative_pooled_prompt_embeds=torch.zeros_like(pooled))
        states.append(dict(latents=lat, timesteps=sched.timesteps, step=0, scheduler=sched, embeds=emb,
                           spec=dict(height=size, width=size, guidance_scale=wl["guidance"], steps=n_steps)))
    img = [(s // 16) ** 2 for s in wl["sizes"] for _ in range(2)]  # CFG: two segments per request
    txt_counts = [wl["text_len"]] * len(img)
    meta = {}

    def step(_):
        meta.update(step_members_once(model, states))
        return None

    _, ms, regions, kregions = _timed(step, None, steps, warmup, model, {"attn_joint"}, breakdown)
    if not all(bool(torch.isfinite(st["latents"]).all()) for st in states):
        raise RuntimeError("sd35 packed: non-finite latents after the timed steps")
    if meta.get("cu_seqlens_img") != build_cu_seqlens(img):
        raise RuntimeError(f"sd35 packed: unexpected segment table {meta.get('cu_seqlens_img')}")
    joint = [n + l for n, l in zip(img, txt_counts)]
    attn_flops = 4.0 * sum(j * j for j in joint) * cfg.dim
    total_flops = step_flops(cfg, img, txt_counts)
    n_img = sum(img)
    out = {
        "metric": wl["metric"], "value": 1000.0 / ms, "unit": "steps/s", "steps": steps, "warmup": warmup,
        "ms_per_step": ms, "tokens_per_s": n_img * 1000.0 / ms,
        "workload": (f"SD3.5-Medium-architecture packed denoise step over 6 requests (2 x 1024^2 + 4 x 512^2), "
                     f"each a CFG pair: 12 joint segments, {n_img} image + {sum(txt_counts)} text tokens, "
                     f"cu_seqlens_img {build_cu_seqlens(img)}, {cfg.layers} blocks, per-request "
                     f"FlowMatch-Euler shift {wl['shift']:g}"),
        "tokens_per_step": sum(joint), "blocks": cfg.layers,
        "model_tflops": total_flops / (ms * 1e-3) / 1e12,
        "model_mfma_frac": total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": _roofline(f"flash_fwd_asm<64, true, true> (joint attention, 12 segments, {sum(joint)} tokens x "
                              f"{cfg.heads} heads)", attn_flops, regions["attn_joint"],
                              algorithmic_bytes=4.0 * sum(joint) * cfg.dim * 2),
        "kernels": _kernel_table(kregions, _sd35_kernel_spec(cfg, img, txt_counts)),
        "reference_a100_ms_per_step": None, "vs_reference_a100": None,
        "reference_context": ("the reference publishes packed SD3.5-M steps of 260.09 ms (1 x 512^2 + 1 x 1024^2) "
                              "and 1003.32 ms (4 x 512^2 + 4 x 1024^2) on one A100-PCIe, results/3.3_Characterization"
                              "_III_Cross-Modal_HBM_Wall_Prompt_Padding_and_Batch_Waste/README.md:32,35; neither is "
                              "this request set"),
        "_img": img, "_cfg": cfg,
    }
    if breakdown:
        out["breakdown_ms_per_step"] = {k: v["total_ms"] / steps for k, v in regions.items()}
    return out


def run_surfaces(repeats=10):
    """GPU time of the reference-shaped entry points against the engine's own
    kernel sequence for the same work, at the Wan2.1 480p CFG-pair shape (2 x 32760
    tokens, 12 heads x 128) and the SD3.5-M 1024^2 CFG-pair joint shape (2 x (4096 +
    333) tokens, 24 heads x 64).  Each figure is the average of `repeats` calls
    bracketed by HIP events on the current stream (host overhead included where a
    call leaves the GPU idle)."""
    import torch

    from ditserve_amd import attention, ops
    from ditserve_amd.wan import fused_qk_norm_rope

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(11)

    def rnd(*shape, scale=1.0):
        return (torch.randn(shape, generator=g, device=dev) * scale).to(torch.bfloat16)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(repeats):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / repeats

    out = {}
    # Wan self-attention of one block: QK-norm + RoPE, V staging, attention
    B, S, H, D = 2, 32760, 12, 128
    qkv = rnd(B * S, 3 * H * D)
    wq = torch.ones(H * D, device=dev)
    cos, sin = torch.ones(1, S, 1, D, device=dev), torch.zeros(1, S, 1, D, device=dev)
    seg = ops.Segments([0, S, 2 * S], dev)
    rope = ops.Rope(cos.reshape(S, D)[:, 0::2].contiguous(), sin.reshape(S, D)[:, 1::2].contiguous(),
                    [(S, 1, 1)] * B, seg, D // 2, 0)
    q, k, v = qkv[:, :H * D], qkv[:, H * D:2 * H * D], qkv[:, 2 * H * D:]

    # the engine's q norm weight carries softmax_scale * log2(e) (the pre-scaled kernel's q)
    wq_pre = wq * (ops.LOG2E / math.sqrt(D))

    def engine():
        ops.qk_norm_rope_(q, k, wq_pre, wq, D, 1e-6, rope=rope)
        vt = ops.transpose_v(v, H, D, seg)
        return ops.flash_attn_varlen(q, k, None, seg, seg, H, D, vt=vt, q_prescaled=True)
    out["wan_self_engine_ms"] = timed(engine)
    qb, kb, vb = (x.reshape(B, S, H * D) for x in (q.contiguous(), k.contiguous(), v.contiguous()))

    def plugin():
        # the reference's processor: slot -> BHSD views -> attention backend -> [B, S, H*D]
        qq, kk = fused_qk_norm_rope(qb, kb, wq, wq, cos, sin, H)
        o, _ = attention.ditk_attention(qq.transpose(1, 2), kk.transpose(1, 2),
                                        vb.view(B, S, H, D).transpose(1, 2), attention.AttnCall())
        return o.transpose(1, 2).flatten(2, 3)
    out["wan_self_reference_surface_ms"] = timed(plugin)
    out["wan_fused_qk_norm_rope_slot_ms"] = timed(lambda: fused_qk_norm_rope(qb, kb, wq, wq, cos, sin, H))
    out["wan_qk_norm_rope_in_place_ms"] = timed(lambda: ops.qk_norm_rope_(q, k, wq, wq, D, 1e-6, rope=rope))
    del qkv, q, k, v, qb, kb, vb
    _release()
    # SD3.5 joint attention: engine (in-place sources) vs the varlen slot on gathered joint rows
    H2, D2, n, l = 24, 64, 4096, 333
    qi, ki, vi = rnd(2 * n, H2 * D2, scale=0.18), rnd(2 * n, H2 * D2), rnd(2 * n, H2 * D2)
    qt, kt, vtx = rnd(2 * l, H2 * D2, scale=0.18), rnd(2 * l, H2 * D2), rnd(2 * l, H2 * D2)
    si, st, sj = ops.Segments([0, n, 2 * n], dev), ops.Segments([0, l, 2 * l], dev), \
        ops.Segments([0, n + l, 2 * (n + l)], dev)

    def joint_engine():
        vt = ops.transpose_v_joint(vi, vtx, H2, D2, si, st, sj)
        return ops.joint_attention_q_prescaled(qi, qt, ki, kt, vt, si, st, sj, H2, D2)
    out["sd35_joint_engine_ms"] = timed(joint_engine)
    cat = lambda a, b: torch.cat([a[:n], b[:l], a[n:], b[l:]]).view(-1, H2, D2)  # noqa: E731
    jq, jk, jv = cat(qi, qt), cat(ki, kt), cat(vi, vtx)
    cu = torch.tensor([0, n + l, 2 * (n + l)], dtype=torch.int32, device=dev)
    out["sd35_varlen_slot_ms"] = timed(lambda: attention.flash_attn_varlen_func(jq, jk, jv, cu, cu, n + l, n + l))
    attention.check_tables()
    return {"metric": "reference-surface entry points vs the engine path (GPU ms per call)", "unit": "ms",
            "higher_is_better": False, "repeats": repeats, **{k: round(v, 4) for k, v in out.items()},
            "workload": "Wan2.1 480p CFG pair (2 x 32760 tokens, 12 x 128) self-attention with QK-norm + RoPE; "
                        "SD3.5-M 1024^2 CFG pair joint attention (2 x (4096 + 333) tokens, 24 x 64)"}


def run_wan_block(repeats=20):
    """One Wan2.1 block on the 1x30x52 grid (1560 tokens, 77 valid text rows, t=500)."""
    import torch

    from ditserve_amd.wan import WanConfig, WanTransformer

    cfg, dev = WanConfig(layers=1), "cuda"
    model = WanTransformer.random(cfg, seed=0, device=dev)
    g = torch.Generator().manual_seed(1)
    lat = torch.randn((16, 1, 60, 104), generator=g).to(dev)
    text = torch.randn((512, 4096), generator=g)
    text[77:] = 0
    packet = model.begin_packed_packet([lat], [500.0], [text.to(dev)])
    h0 = packet["hidden"].clone()
    for _ in range(3):
        packet["hidden"] = h0.clone()
        model.forward_block(packet, 0)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    inputs = [h0.clone() for _ in range(repeats)]
    start.record()
    for x in inputs:
        packet["hidden"] = x
        model.forward_block(packet, 0)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / repeats
    return {"metric": "Wan2.1 block forward ms (1560 tokens)", "value": ms, "unit": "ms/block",
            "higher_is_better": False, "steps": repeats, "warmup": 3, "tokens_per_s": 1560 * 1000.0 / ms,
            "workload": "one Wan2.1-T2V-1.3B-architecture block, grid 1x30x52 (1560 tokens), 512 text rows "
                        "(77 valid), t = 500, bf16"}


def _public(d):
    return {k: v for k, v in d.items() if not k.startswith("_")}


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); this build "
              "has no multi-GPU path", file=sys.stderr)
        sys.exit(2)
    import torch

    if args.surfaces:
        print(json.dumps(run_surfaces()), flush=True)
        return
    threads = cpu_threads()
    cpu = not args.no_cpu_baseline

    def headline_for(name, steps, warmup):
        if name == "sd35_medium_1024":
            return run_sd35(steps, warmup, args.breakdown)
        if name == "sd35_packed_2x1024_4x512":
            return run_sd35_packed(steps, warmup, args.breakdown)
        if name == "wan21_packed_4req":
            return run_wan_packed(steps, warmup, args.breakdown)
        return run_wan_cfg(name, steps, warmup, args.breakdown)

    def cpu_for(name, res):
        torch.set_num_threads(threads)
        if name == "sd35_medium_1024":
            return cpu_baseline_sd35(res["_cfg"], res["_n_img"], WORKLOADS[name]["text_len"], threads)
        if name == "sd35_packed_2x1024_4x512":
            wl = WORKLOADS[name]
            return cpu_baseline_sd35_packed(res["_cfg"], wl["sizes"], wl["text_len"], threads)
        if name == "wan21_packed_4req":
            from ditserve_amd.wan import WAN21_T2V_1_3B
            return cpu_baseline_wan_packed(WAN21_T2V_1_3B, res["_grids"], threads)
        label = "Wan2.1" if WORKLOADS[name]["arch"] == "wan21" else "Wan2.2-5B"
        return cpu_baseline_wan_step(res["_cfg"], res["_grid"], threads, label)

    head = headline_for(args.workload, args.steps, args.warmup)
    calibration_copy()
    print(f"[bench] {args.workload}: {head['ms_per_step']:.2f} ms/step over {args.steps} steps", file=sys.stderr,
          flush=True)
    out = {
        "metric": head["metric"], "value": head["value"], "unit": head["unit"], "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": head["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": head["vs_reference_a100"], "dtype": "bf16",
        "data": "synthetic: random-init weights N(0,0.02^2), latent/text N(0,1)",
        "config": {"workload": head["workload"], "tokens_per_step": head["tokens_per_step"],
                   "blocks": head["blocks"]},
        "tokens_per_s": head["tokens_per_s"], "model_tflops": head["model_tflops"],
        "model_mfma_frac": head["model_mfma_frac"], "roofline": head["roofline"], "kernels": head["kernels"],
        "reference_a100_ms_per_step": head["reference_a100_ms_per_step"],
    }
    if "breakdown_ms_per_step" in head:
        out["breakdown_ms_per_step"] = head["breakdown_ms_per_step"]
    if cpu:
        out["cpu_baseline"] = cpu_for(args.workload, head)
    if not args.no_per_config:
        per = {}
        plan = [("wan21_480p", 3, 1), ("wan21_packed_4req", 5, 2), ("sd35_medium_1024", 10, 3),
                ("sd35_packed_2x1024_4x512", 5, 2), ("wan22_ti2v_5b_704p", 3, 1), ("wan21_720p", 2, 1),
                ("wan21_480p_33f", 5, 2)]
        for name, steps, warmup in plan:
            if name == args.workload:
                res = dict(head)
                if cpu:
                    res["cpu_baseline"] = out["cpu_baseline"]
            else:
                _release()
                res = headline_for(name, steps, warmup)
                if cpu:
                    res["cpu_baseline"] = cpu_for(name, res)
            key = {"wan21_480p": "wan21_480p_cfg2", "wan21_packed_4req": "wan21_packed_4req",
                   "sd35_medium_1024": "sd35_medium_1024_cfg2",
                   "sd35_packed_2x1024_4x512": "sd35_packed_2x1024_4x512_cfg2",
                   "wan22_ti2v_5b_704p": "wan22_ti2v_5b_704p_cfg2", "wan21_720p": "wan21_720p_cfg2",
                   "wan21_480p_33f": "wan21_480p_33f_cfg2"}[name]
            res.pop("breakdown_ms_per_step", None)
            per[key] = _public(res)
            print(f"[bench] {key}: {res['ms_per_step']:.2f} ms/step", file=sys.stderr, flush=True)
        _release()
        blk = run_wan_block()
        if cpu:
            from ditserve_amd.wan import WAN21_T2V_1_3B
            torch.set_num_threads(threads)
            blk["cpu_baseline"] = cpu_baseline_wan_block(WAN21_T2V_1_3B, threads)
            blk["gpu_vs_cpu"] = blk["cpu_baseline"]["value"] / blk["value"]
        per["wan21_block_1560tok"] = blk
        out["per_config"] = per
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

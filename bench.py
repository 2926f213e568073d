#!/usr/bin/env python3
"""Benchmark: one Wan2.1-T2V-1.3B denoise step at 480x832x81 frames with CFG batch 2
(2 x 32760 tokens), bf16, on one MI355X.

A step = packed prelude for the (cond, uncond) pair + 30 DiT blocks + prediction
+ the fused CFG combine and UniPC update (Wan's scheduler recipe: flow sigmas,
shift 3.0, 50-step schedule, order 2 with corrector), all on the ditk HIP kernels.
The model timestep of each step is the schedule's (999, 997, ...).
Synthetic data: random-init weights N(0, 0.02^2) (norm weights N(1, 0.02^2)),
latent 16x21x60x104 N(0,1), text contexts 512x4096 N(0,1) with 120 (cond) and 0
(uncond) valid rows.

Prints one JSON line (rank 0).  `roofline` is for the dominant kernel, the
self-attention flash kernel, from HIP events recorded on its launch stream over
the timed steps.  `cpu_baseline` times the oracle (CPU fp32 restatement of the
reference block) on one full-shape block-forward and extrapolates x60.
"""
import argparse
import json
import os
import sys
import time

METRIC = "denoise steps/s & tokens/s, Wan2.1-1.3B 480p-81f CFG2; attn % bf16 MFMA peak"
PEAK_BF16_TFLOPS = 2500.0
LATENT = (16, 21, 60, 104)
TEXT_VALID = (120, 0)
GUIDANCE = 5.0
FLOW_SHIFT = 3.0
SCHEDULE_STEPS = 50
CALIB_BYTES = 256 << 20
# A100-PCIe-40GB, fp16, same workload: 3964.62 ms per step (the reference's published figure)
REFERENCE_STEPS_PER_S = 1000.0 / 3964.62
# HBM traffic of one self-attention launch, from two rocprofv3 --pmc passes over this
# bench (FETCH_SIZE, then WRITE_SIZE, KiB per dispatch), each scaled by that counter's
# reading for the CALIB_BYTES copy: FETCH 917467.5 KiB x 1.9997, WRITE 196581.8 KiB x 1.0000
# (profiles/wan21_480p_cfg2_step_traffic.md).  Re-measure after kernel changes.
ATTN_SELF_TRAFFIC_BYTES = (917548 * 1.9997 + 196607 * 1.0000) * 1024


# Other single-GPU workloads of the same step (reported per config; the default
# line is the headline): A100-PCIe reference step times for the same shapes.
WORKLOADS = {
    "wan21_480p": None,
    "wan22_ti2v_5b_704p": dict(latent=(48, 31, 44, 80), text_valid=(150, 0), flow_shift=5.0, ref_ms=7813.18),
    "sd35_medium_1024": dict(latent=(16, 128, 128), text_len=333, steps=28, shift=3.0, ref_ms=217.23),
}


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--breakdown", action="store_true", help="per-op HIP-event breakdown in the JSON")
    ap.add_argument("--workload", default="wan21_480p", choices=sorted(WORKLOADS),
                    help="wan21_480p (the headline line), wan22_ti2v_5b_704p or sd35_medium_1024")
    return ap.parse_args()


def cpu_baseline(seq=32760, grid=(21, 30, 52)):
    """Oracle (CPU fp32, the reference block arithmetic on PyTorch CPU ops) on one
    full-shape Wan2.1 block-forward; steps/s extrapolated over 30 blocks x 2 branches."""
    import torch

    from ditserve_amd.wan import WanConfig, random_state_dict
    from oracle import common as oc
    from oracle import wan as ow

    threads = min(os.cpu_count() or 1, 16)
    torch.set_num_threads(threads)
    cfg = WanConfig(layers=1)
    sd = random_state_dict(cfg, seed=0)
    g = torch.Generator().manual_seed(2)
    h = torch.randn(seq, cfg.dim, generator=g)
    enc = torch.randn(cfg.text_len, cfg.dim, generator=g)
    proj = torch.randn(6, cfg.dim, generator=g) * 0.02
    cos, sin = ow.rope_freqs(grid)
    # warm-up on a small slice, then one timed full-shape block
    ow.block_forward(sd, 0, h[:1560], enc, proj, cos[:1560], sin[:1560], cfg.heads, attn=oc.sdpa_fast)
    t0 = time.perf_counter()
    ow.block_forward(sd, 0, h, enc, proj, cos, sin, cfg.heads, attn=oc.sdpa_fast)
    block_s = time.perf_counter() - t0
    step_s = block_s * cfg.layers * 2
    return {
        "value": 1.0 / step_s,
        "unit": "steps/s",
        "cores": threads,
        "kind": "port",
        "sample": f"1 Wan2.1 block-forward at S={seq} (one CFG branch), fp32, CPU flash SDPA: "
                  f"{block_s:.2f} s; extrapolated x60 (30 blocks x 2 branches)",
        "tokens_per_s": 2 * seq / step_s,
    }


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); this build "
              "has no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    if args.workload == "sd35_medium_1024":
        return run_sd35(args)

    import torch

    from ditserve_amd.profiling import EventProfiler
    from ditserve_amd.solver import UniPCFlowScheduler
    from ditserve_amd.wan import WAN21_T2V_1_3B, WAN22_TI2V_5B, WanTransformer, step_flops

    wl = WORKLOADS[args.workload]
    cfg = WAN21_T2V_1_3B if wl is None else WAN22_TI2V_5B
    latent_shape = LATENT if wl is None else wl["latent"]
    text_valid = TEXT_VALID if wl is None else wl["text_valid"]
    flow_shift = FLOW_SHIFT if wl is None else wl["flow_shift"]
    ref_steps_per_s = REFERENCE_STEPS_PER_S if wl is None else 1000.0 / wl["ref_ms"]
    dev = "cuda"
    model = WanTransformer.random(cfg, seed=0, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    latent = torch.randn(latent_shape, generator=g, device=dev)
    texts = []
    for valid in text_valid:
        t = torch.randn((cfg.text_len, cfg.text_dim), generator=g, device=dev)
        t[valid:] = 0
        texts.append(t)
    seq = (latent_shape[1] // cfg.patch[0]) * (latent_shape[2] // cfg.patch[1]) * (latent_shape[3] // cfg.patch[2])
    # calibration buffers for HBM-traffic counters: a plain copy of exactly
    # CALIB_BYTES, run once after the timed steps (cold by then), outside timing
    calib_src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    calib_dst = torch.empty_like(calib_src)

    sched = UniPCFlowScheduler(flow_shift=flow_shift)
    sched.set_timesteps(max(SCHEDULE_STEPS, args.warmup + args.steps))

    def step(lat):
        t = float(sched.timesteps[sched.step_index])
        cond, uncond = model.forward_packed([lat, lat], [t, t], texts)
        return sched.step(cond, t, lat, uncond=uncond, guidance=GUIDANCE)[0]

    for _ in range(args.warmup):
        latent = step(latent)
    torch.cuda.synchronize()

    # only the roofline kernel's region is timed unless the breakdown is asked for
    prof = EventProfiler(enabled=True, only=None if args.breakdown else {"attn_self"})
    model.profiler = prof
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        latent = step(latent)
    end.record()
    torch.cuda.synchronize()
    model.profiler = EventProfiler(enabled=False)
    if not bool(torch.isfinite(latent).all()):
        raise RuntimeError("non-finite latent after the timed steps")
    calib_dst.copy_(calib_src)  # the known-size copy the traffic counters are scaled by
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    regions = prof.summary()

    attn = regions["attn_self"]
    attn_flops = 4.0 * 2 * seq * seq * cfg.dim  # per launch: 2 segments (CFG pair), non-causal
    attn_tflops = attn_flops / (attn["avg_ms"] * 1e-3) / 1e12
    total_flops = step_flops(cfg, [seq, seq], cfg.text_len)

    out = {
        "metric": METRIC,
        "value": 1000.0 / ms,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (1000.0 / ms) / ref_steps_per_s,
        "dtype": "bf16",
        "data": "synthetic: random-init weights N(0,0.02^2), latent/text N(0,1)",
        "config": {"workload": (
                       "Wan2.1-T2V-1.3B-architecture denoise step, latent 16x21x60x104 (480x832x81f), "
                       "CFG pair packed as 2 x 32760 tokens, 30 blocks, text 512 (valid 120/0), UniPC flow-shift-3 "
                       "50-step schedule (t = 999, 997, ...)") if wl is None else (
                       f"Wan2.2-TI2V-5B-architecture denoise step, latent {'x'.join(map(str, latent_shape))} "
                       f"(704x1280x121f), CFG pair packed as 2 x {seq} tokens, {cfg.layers} blocks, text 512 "
                       f"(valid {text_valid[0]}/{text_valid[1]}), UniPC flow-shift-{flow_shift:g} 50-step schedule"),
                   "tokens_per_step": 2 * seq, "blocks": cfg.layers},
        "tokens_per_s": 2 * seq * 1000.0 / ms,
        "model_tflops": total_flops / (ms * 1e-3) / 1e12,
        "model_mfma_frac": total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": {
            "kernel": f"flash_fwd_kernel<128> (self-attention, 2 x {seq} tokens x {cfg.heads} heads)",
            "bound": "mfma",
            "achieved": attn_tflops,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": attn_tflops / PEAK_BF16_TFLOPS,
            "traffic": ATTN_SELF_TRAFFIC_BYTES if wl is None else None,
            "traffic_unit": "bytes/launch",
            "algorithmic_bytes": 4.0 * 2 * seq * cfg.dim * 2,
            "avg_launch_ms": attn["avg_ms"],
            "launches": attn["count"],
            "flops_per_launch": attn_flops,
        },
        "reference_a100_steps_per_s": ref_steps_per_s,
    }
    if args.breakdown:
        out["breakdown_ms_per_step"] = {k: v["total_ms"] / args.steps for k, v in regions.items()}
    if not args.no_cpu_baseline and wl is None:
        out["cpu_baseline"] = cpu_baseline(seq)
    print(json.dumps(out), flush=True)


def run_sd35(args):
    """SD3.5-Medium 1024^2 denoise step, CFG as a packed pair of joint
    segments (4096 image + 333 text tokens each), 24 blocks, FlowMatch-Euler."""
    import torch

    from ditserve_amd.profiling import EventProfiler
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
    sched.set_timesteps(max(wl["steps"], args.warmup + args.steps))
    n_img = (wl["latent"][1] // cfg.patch) * (wl["latent"][2] // cfg.patch)
    n_joint = n_img + wl["text_len"]

    def step(lat):
        t = float(sched.timesteps[sched.step_index])
        outs, _ = forward_packed_sd35(torch, model, [lat.unsqueeze(0)] * 2, [t, t],
                                      [text_u.unsqueeze(0), text_c.unsqueeze(0)], [pooled_u, pooled_c])
        return sched.step(outs[1], t, lat, uncond=outs[0], guidance=7.0)[0]

    for _ in range(args.warmup):
        latent = step(latent)
    torch.cuda.synchronize()
    prof = EventProfiler(enabled=True, only=None if args.breakdown else {"attn_joint"})
    model.profiler = prof
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        latent = step(latent)
    end.record()
    torch.cuda.synchronize()
    model.profiler = EventProfiler(enabled=False)
    if not bool(torch.isfinite(latent).all()):
        raise RuntimeError("non-finite latent after the timed steps")
    ms = start.elapsed_time(end) / args.steps
    regions = prof.summary()
    attn = regions["attn_joint"]
    attn_flops = 4.0 * 2 * n_joint * n_joint * cfg.dim
    attn_tflops = attn_flops / (attn["avg_ms"] * 1e-3) / 1e12
    total_flops = step_flops(cfg, [n_img, n_img], [wl["text_len"]] * 2)
    out = {
        "metric": METRIC, "value": 1000.0 / ms, "unit": "steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": (1000.0 / ms) / (1000.0 / wl["ref_ms"]), "dtype": "bf16",
        "data": "synthetic: random-init weights N(0,0.02^2), latent/text/pooled N(0,1), uncond zeros",
        "config": {"workload": f"SD3.5-Medium-architecture denoise step at 1024x1024 (latent 16x128x128), CFG pair "
                               f"packed as 2 x ({n_img} image + {wl['text_len']} text) joint tokens, {cfg.layers} blocks "
                               f"(13 with dual attention), FlowMatch-Euler shift {wl['shift']:g}",
                   "tokens_per_step": 2 * n_joint, "blocks": cfg.layers},
        "tokens_per_s": 2 * n_img * 1000.0 / ms,
        "model_tflops": total_flops / (ms * 1e-3) / 1e12,
        "model_mfma_frac": total_flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
        "roofline": {"kernel": f"flash_fwd_kernel<64> (joint attention, 2 x {n_joint} tokens x {cfg.heads} heads)",
                     "bound": "mfma", "achieved": attn_tflops, "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": attn_tflops / PEAK_BF16_TFLOPS, "traffic": None, "avg_launch_ms": attn["avg_ms"],
                     "launches": attn["count"], "flops_per_launch": attn_flops},
        "reference_a100_steps_per_s": 1000.0 / wl["ref_ms"],
    }
    if args.breakdown:
        out["breakdown_ms_per_step"] = {k: v["total_ms"] / args.steps for k, v in regions.items()}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

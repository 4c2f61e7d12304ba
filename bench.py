"""MoE-layer forward benchmark on one MI355X (the BASELINE.json metric).

python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--no-cpu] [--no-train]

A step is one MoE-layer forward (router, dispatch, grouped SwiGLU GEMMs,
combine, aux losses; train mode so the aux loss is computed) over one batch of
synthetic input already resident in HBM.  Rank 0 prints one JSON line with
whole-job tokens/s (timed with nothing but the forwards on the stream, plus a HIP
event pair around the gate/up grouped GEMM on every EVENT_EVERY-th forward: the
roofline of that dominant kernel), per-stage figures from a separate pass
and a CPU baseline (the op-for-op torch-CPU port of the reference path, timed on this
host on a bounded token sample).  Token-choice bf16 configs also report a
"training" object: the training forward + backward step on the HIP kernels,
timed in its own pass after the forward metric's timed region.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "kolmogorov-moe-architecture_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE-layer fwd tokens/sec (d2048,16e,top-2,bf16); % MFMA peak; dispatch GB/s"
PEAK_BF16 = 2.5e15
PEAK_FP8 = 5.0e15
PEAK_HBM = 8.0e12
EVENT_EVERY = 5  # timed forwards per sampled gate/up event pair
NEAR_TIE = 2.0 ** -16  # router logit gap counted as a near-tie


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=[2, 3, 4, 5])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-train", action="store_true", help="skip the training-step (backward) pass")
    ap.add_argument("--no-block", action="store_true",
                    help="skip the fused FFN-block (RMSNorm + MoE + residual) pass")
    ap.add_argument("--settle-ms", type=float, default=250.0,
                    help="after the warm-up steps and the routing statistics, keep running untimed forwards for "
                         "this much wall time, right up to the timed region, so that it starts at the settled clock")
    ap.add_argument("--stage-steps", type=int, default=20, help="forwards of the per-stage timing pass")
    ap.add_argument("--cpu-tokens", type=int, default=2048, help="token sample of the CPU baseline")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run a plain 512 MiB device copy (the reference for PMC byte-counter scaling)")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations' summary (the 'configs' object)")
    ap.add_argument("--config-steps", type=int, default=20, help="timed forwards per other configuration")
    ap.add_argument("--no-library-gemm", dest="library_gemm", action="store_false",
                    help="skip the vendor-library dense GEMM reference (library_gemm)")
    return ap.parse_args()


def stage_bytes_flops(wl, layer, fwd_state):
    """Algorithmic work per launch of each stage (bytes or FLOPs)."""
    d, F, E, k = wl.d, wl.F, wl.E, wl.k
    s = 2  # bf16
    T = wl.T
    a_kept = fwd_state["a_kept"]
    a_all = fwd_state["a_all"]
    t_in = fwd_state["t_in"]
    xs = 1 if wl.fp8 else s
    return {
        "gemm_gate_up": ("flop", 4.0 * d * F * a_kept),
        "gemm_down": ("flop", 2.0 * d * F * a_kept),
        # fp8: read each routed token row once, write its kept quantised rows + scales;
        # bf16: tables only (the gate/up GEMM gathers the rows): read ids twice (8 B) and
        # weights (4 B), write row_token / slot_row / slot_w (12 B) per assignment
        "dispatch": ("byte", t_in * d * s + a_kept * d * xs + 8.0 * a_all + a_kept * 4 if wl.fp8
                     else 28.0 * a_all),
        "gather": ("byte", a_kept * d * s + a_kept * d * xs + 4.0 * a_kept),
        # read the kept expert rows, write y, 8 B/assignment of metadata
        "combine": ("byte", a_kept * d * s + T * d * s + 8.0 * a_all),
        "router": ("byte", t_in * d * s + t_in * E * 4 + t_in * k * 12),
    }


def run_gpu(args, wl, light=False):
    """The forward metric of workload `wl` (timed region, per-stage pass); unless `light`,
    also the materialising-dispatch, training and FFN-block passes."""
    import torch
    from kmoe import ops, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t = synth.make_tensors(wl, "cpu")
    t = {kk: v.to(dev) for kk, v in t.items()}
    layer = synth.build_layer(wl, dev, t).train()
    x = t["x"]
    torch.cuda.synchronize()

    def step():
        return layer(x)

    with torch.no_grad():
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        # routing statistics of this input (outside the timed region)
        moe = layer.ffn if wl.mod else layer
        if wl.routing == "expert_choice":
            C = moe.router.capacity(wl.S)
            a_all = a_kept = wl.E * wl.B * min(C, wl.S)
            t_in = wl.T
        else:
            counts = moe.last_expert_counts.cpu().long()
            t_in = wl.B * layer.ffn_mod_router.keep_count(wl.S) if wl.mod else wl.T
            a_all = t_in * wl.k
            if moe.drop_overflow:
                cap = ops.capacity_of(moe.capacity_factor, t_in, wl.k, wl.E)
                a_kept = int(counts.clamp(max=cap).sum())
            else:
                a_kept = int(counts.sum())
        # routing conditioning of this input: tokens whose k-th and (k+1)-th largest fp32
        # logits are within NEAR_TIE of each other (there the top-k choice can flip under
        # a different fp32 summation order of the router's dot products; exact ties go to
        # the lower expert index)
        near = None
        if wl.routing != "expert_choice":
            xr = x.reshape(wl.T, wl.d)
            if wl.mod:
                xr = xr[layer.ffn_mod_router.select(x).token_rows.long()]
            lg = moe.router.route(xr).logits  # (with the logit bias, as the kernel routes on)
            top = torch.topk(lg, wl.k + 1, dim=-1).values
            gap = top[:, wl.k - 1] - top[:, wl.k]
            near = {"tokens": int((gap <= NEAR_TIE).sum()), "exact_ties": int((gap == 0).sum()),
                    "of": int(lg.shape[0]), "threshold": NEAR_TIE,
                    "note": "tokens whose k-th and (k+1)-th largest router logits differ by at most the threshold"}
        # clock settle: the GPU's clock ramps over the first tens of milliseconds of load
        # (5 warm-up forwards left the gate/up GEMM ~9% slower than at the settled clock),
        # so untimed forwards continue for settle_ms of wall time.  They run
        # right up to the timed region: an idle gap before it (host-side statistics) let the
        # clock overshoot, and the first timed forwards then ran ~30% slower
        settle = 0
        t_w = time.perf_counter()
        while (time.perf_counter() - t_w) * 1e3 < args.settle_ms:
            for _ in range(10):
                step()
            settle += 10
            torch.cuda.synchronize()
        # timed region: K back-to-back forwards; the only extra work on the stream is
        # a HIP event pair around the gate/up GEMM launch (the roofline kernel) on
        # every EVENT_EVERY-th forward (an event pair costs ~6 us of drain per event
        # on this GPU, so it is sampled rather than put on every forward)
        timed = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            ops.set_stage_timing(timed if i % EVENT_EVERY == 0 else None, only={"gemm_gate_up"})
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ops.set_stage_timing(None)
        # the materialising dispatch (tables + the row copy; what the fp8 path and
        # the C-ABI's xperm output use), outside the timed region, on this routing
        rows_us = None
        if not light and not wl.fp8 and wl.routing != "expert_choice" and not wl.mod:
            r0 = moe.router.route(x.reshape(wl.T, wl.d))
            cap = ops.capacity_of(moe.capacity_factor, wl.T, wl.k, wl.E) if moe.drop_overflow else 0
            for _ in range(3):
                ops.dispatch(x.reshape(wl.T, wl.d), r0.idx, r0.w, wl.E, capacity=cap, block_counts=r0.block_counts)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            # the GPU spins ~1.5 ms first, so that the host has enqueued every launch
            # before e0 fires: the pair then times the kernels back to back (as inside a
            # training step, where the host runs ahead), not the host's launch overhead
            torch.cuda._sleep(3_000_000)
            e0.record()
            for _ in range(10):
                ops.dispatch(x.reshape(wl.T, wl.d), r0.idx, r0.w, wl.E, capacity=cap, block_counts=r0.block_counts)
            e1.record()
            torch.cuda.synchronize()
            rows_us = e0.elapsed_time(e1) / 10 * 1e3
        # per-stage breakdown in a separate pass: an event pair around every stage
        # (their host-side cost would distort the timed region of small configs)
        events = []
        ops.set_stage_timing(events)
        for _ in range(args.stage_steps):
            step()
        torch.cuda.synchronize()
        ops.set_stage_timing(None)
    stages = {}
    for name, a, b in events:
        stages.setdefault(name, []).append(a.elapsed_time(b) * 1e3)  # us
    gu_timed = [a.elapsed_time(b) * 1e3 for _, a, b in timed]
    work = stage_bytes_flops(wl, layer, dict(a_kept=a_kept, a_all=a_all, t_in=t_in))
    stage_out = {}
    for name, v in stages.items():
        # median: a one-off host stall (an allocation) inside one event pair of the
        # pass would otherwise dominate a mean
        us = statistics.median(v)
        rec = {"us": round(us, 2), "launches_per_step": len(v) // args.stage_steps}
        if name in work:
            kind, amount = work[name]
            if kind == "flop":
                rec["TFLOPs"] = round(amount / (us * 1e-6) / 1e12, 1)
                rec["frac_peak"] = round(amount / (us * 1e-6) / (PEAK_FP8 if wl.fp8 else PEAK_BF16), 4)
            else:
                rec["GBps"] = round(amount / (us * 1e-6) / 1e9, 1)
                rec["frac_hbm"] = round(amount / (us * 1e-6) / PEAK_HBM, 4)
        stage_out[name] = rec
    elapsed = t1 - t0
    training = None
    if not light and not (wl.fp8 or wl.mod or wl.routing == "expert_choice") and not args.no_train:
        training = run_training(args, wl, layer, x)
    block = None
    if not light and not (wl.fp8 or wl.mod or wl.routing == "expert_choice") and not args.no_block:
        block = run_block(args, wl, layer, x)
    del layer, t, x
    torch.cuda.empty_cache()
    return dict(elapsed=elapsed, stages=stage_out, a_kept=a_kept, a_all=a_all, t_in=t_in, settle=settle, near_ties=near,
                gemm_us=statistics.mean(gu_timed) if gu_timed else float("nan"), gemm_samples=len(gu_timed),
                work=work, rows_us=rows_us, training=training, block=block)


def config_summary(wl, res, steps):
    """Tokens/s and roofline fractions of one configuration's forward."""
    peak = PEAK_FP8 if wl.fp8 else PEAK_BF16
    st = res["stages"]
    out = {"workload": wl.name, "dtype": "fp8_e4m3" if wl.fp8 else "bf16", "tokens": wl.T,
           "tokens_into_moe": res["t_in"], "assignments": res["a_all"], "assignments_kept": res["a_kept"],
           "steps": steps, "tokens_per_s": round(wl.T * steps / res["elapsed"], 1),
           "ms_per_step": round(res["elapsed"] / steps * 1e3, 4)}
    us = res["gemm_us"]
    if us == us:  # not NaN
        out["gate_up_frac_peak"] = round(res["work"]["gemm_gate_up"][1] / (us * 1e-6) / peak, 4)
        out["gate_up_launch_us"] = round(us, 2)
    g_us = st.get("gemm_gate_up", {}).get("us", 0) + st.get("gemm_down", {}).get("us", 0)
    if g_us:
        fl = res["work"]["gemm_gate_up"][1] + res["work"]["gemm_down"][1]
        out["gemm_TFLOPs"] = round(fl / (g_us * 1e-6) / 1e12, 1)
        out["gemm_frac_peak"] = round(fl / (g_us * 1e-6) / peak, 4)
        out["peak_TFLOPs"] = peak / 1e12
    for name in ("router", "dispatch", "gather", "combine"):
        if name in st and "GBps" in st[name]:
            out[name] = {"us": st[name]["us"], "GBps": st[name]["GBps"], "frac_hbm": st[name]["frac_hbm"]}
    out["stages_us"] = {k: v["us"] for k, v in st.items()}
    if res.get("near_ties") is not None:
        out["near_ties"] = {k: v for k, v in res["near_ties"].items() if k != "note"}
    return out


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def run_block(args, wl, layer, x):
    """The FFN half of the transformer block, out = h + MoE(RMSNorm(h)) (layers.py:142-147,
    184-187), in inference: fused (norm folded into the router and the gate/up GEMM,
    residual add in the combine) against the unfused composition (the reference's
    RMSNorm formula in torch, the same kmoe layer, a torch add).  Timed outside the
    forward metric's region, K forwards between synchronisations."""
    import torch
    from kmoe import ops
    from kmoe.block import MoEFFNBlock

    blk = MoEFFNBlock(layer.config, 0, ffn=layer)
    g = torch.Generator().manual_seed(wl.seed + 200)
    blk.ffn_norm.weight = torch.nn.Parameter((1.0 + 0.1 * torch.randn(wl.d, generator=g)).to(x.device, x.dtype))
    blk.eval()
    norm = blk.ffn_norm
    fns = {"fused": lambda: blk(x), "unfused": lambda: x + layer(norm(x))}
    steps = max(1, args.steps // 2)
    ms = {}
    with torch.no_grad():
        for name, fn in fns.items():
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                fn()
            torch.cuda.synchronize()
            ms[name] = (time.perf_counter() - t0) / steps * 1e3
        events = []
        ops.set_stage_timing(events)
        for _ in range(10):
            fns["fused"]()
        torch.cuda.synchronize()
        ops.set_stage_timing(None)
    assert blk.last_path == "fused"
    layer.train()
    training = run_block_training(args, wl, layer, x, blk.ffn_norm.weight)
    per = {}
    for name, a, b in events:
        per.setdefault(name, []).append(a.elapsed_time(b) * 1e3)
    stages = {name: round(statistics.median(v), 2) for name, v in per.items()}
    return {"fused_ms": round(ms["fused"], 4), "unfused_ms": round(ms["unfused"], 4),
            "fused_tokens_per_s": round(wl.T / (ms["fused"] * 1e-3), 1),
            "unfused_tokens_per_s": round(wl.T / (ms["unfused"] * 1e-3), 1),
            "saved_us": round((ms["unfused"] - ms["fused"]) * 1e3, 1), "steps": steps,
            "fused_stages_us": stages, "training": training,
            "note": "h + MoE(RMSNorm(h)), eval, bf16 norm weight; unfused = torch RMSNorm (embeddings.py:190-195) "
                    "+ kmoe layer + torch add"}


def run_block_training(args, wl, layer, x, norm_w):
    """Training steps of the FFN half of the block through autograd (forward, then
    backward of sum(out * dy) + aux to h and every parameter), in training mode with
    the default residual dropout 0.1: with the MoD router (the reference's default mod_enabled,
    layers.py:148-185) and without.  Gradients are set to None before each step (as an
    optimizer's zero_grad does); the parameters do not change, so the packed weights
    stay cached (with_repack: new parameter versions every step, as after an update)."""
    import dataclasses

    import torch
    from kmoe import ops
    from kmoe.block import MoEFFNBlock

    out = {}
    g = torch.Generator().manual_seed(wl.seed + 300)
    dy = torch.randn(wl.B, wl.S, wl.d, generator=g).to(torch.bfloat16).to(x.device)
    h = x.detach().clone().requires_grad_(True)
    one = torch.ones((), device=x.device)
    steps = max(1, args.steps // 5)
    for mod in (True, False):
        # the reference's default residual dropout (config.py:87): the fused path applies
        # its keep mask in the combine
        cfg = dataclasses.replace(layer.config, mod_enabled=mod, residual_dropout=0.1)
        blk = MoEFFNBlock(cfg, 0, ffn=layer).to(x.device)
        blk.ffn_norm.weight = torch.nn.Parameter(norm_w.detach().clone())
        if mod:
            blk.ffn_mod_router.to(x.device, torch.bfloat16)
        blk.train()
        params = [p_ for p_ in blk.parameters()]

        def step(repack=False):
            for p_ in params:
                p_.grad = None
                if repack:
                    torch.autograd.graph.increment_version(p_)
            h.grad = None
            o = blk(h)
            torch.autograd.backward([o, blk.aux_loss], [dy, one])

        for _ in range(3):
            step()
        assert blk.last_path == "fused_train"
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(steps):
            step(repack=True)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        events = []
        ops.set_stage_timing(events)
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        ops.set_stage_timing(None)
        per = {}
        for name, a, b in events:
            per[name] = per.get(name, 0.0) + a.elapsed_time(b) * 1e3 / steps
        key = "mod" if mod else "no_mod"
        out[key] = {"step_ms": round((t1 - t0) / steps * 1e3, 3),
                    "tokens_per_s": round(wl.T * steps / (t1 - t0), 1),
                    "step_ms_with_repack": round((t2 - t1) / steps * 1e3, 3),
                    "stages_us": {n: round(v, 1) for n, v in per.items()}}
        if mod:
            out[key]["kept_tokens"] = wl.B * blk.ffn_mod_router.keep_count(wl.S)
        layer.zero_grad(set_to_none=True)
        del blk
    out["steps"] = steps
    out["note"] = ("autograd step of out = h + MoE(RMSNorm(h)) (MoD-gated: the kept tokens only, "
                   "mod_capacity_factor 0.75), loss sum(out * dy) + aux, training mode, residual dropout 0.1 "
                   "(a fresh Bernoulli keep mask per step, applied in the combine)")
    return out


def run_training(args, wl, layer, x):
    """One training step of the layer (the forward that keeps what the backward needs,
    then the backward on the HIP kernels), timed outside the forward metric's region:
    K steps between synchronisations, then a per-stage pass with an event pair around
    every stage (us per step, summed over the stage's launches)."""
    import torch
    from kmoe import backward as BW, ops

    T, d, F, k = wl.T, wl.d, wl.F, wl.k
    x2d = x.reshape(T, d)
    dev = x2d.device
    g = torch.Generator().manual_seed(wl.seed + 100)
    dy = torch.randn(T, d, generator=g).to(torch.bfloat16).to(dev)
    ga = torch.ones((), device=dev, dtype=torch.float32)
    w_out = layer.router.router[2].weight
    bw = layer._bwd_weights()

    ge = layer.grouped_experts
    params = (ge.w1, ge.w2, ge.w3, layer.router.router[0].weight)

    def train_step():
        _, _, sv = layer._train_forward(x2d, T, torch.bfloat16)
        return BW.moe_backward(sv, dy, ga, w_out, bw, wl.E, F, layer.load_balance_loss_weight,
                               layer.router_z_loss_weight)

    def train_step_repack():
        # what an optimizer step leaves behind: new parameter versions, so the forward and
        # backward packed weights are rebuilt (the version bump touches no data; the
        # optimizer's own update is not part of the layer's step)
        for p_ in params:
            torch.autograd.graph.increment_version(p_)
        bw_ = layer._bwd_weights()
        _, _, sv = layer._train_forward(x2d, T, torch.bfloat16)
        return BW.moe_backward(sv, dy, ga, w_out, bw_, wl.E, F, layer.load_balance_loss_weight,
                               layer.router_z_loss_weight)

    steps = max(1, args.steps // 5)
    with torch.no_grad():
        for _ in range(3):
            train_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            train_step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        for _ in range(2):
            train_step_repack()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        for _ in range(steps):
            train_step_repack()
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        events = []
        ops.set_stage_timing(events)
        for _ in range(steps):
            train_step()
        torch.cuda.synchronize()
        ops.set_stage_timing(None)
    per = {}
    for name, a, b in events:
        per[name] = per.get(name, 0.0) + a.elapsed_time(b) * 1e3 / steps
    a_kept = int(layer.last_expert_counts.clamp(
        max=ops.capacity_of(layer.capacity_factor, T, k, wl.E) if layer.drop_overflow else 1 << 30).sum().item())
    dF = 2.0 * d * F * a_kept
    gemm = {"bwd_gemm_dh": dF, "bwd_gemm_dx": 2 * dF, "bwd_wgrad_w3": dF, "bwd_wgrad_w13": 2 * dF,
            "bwd_wgrad_router": 2.0 * T * 128 * d, "gemm_gate_up": 2 * dF, "gemm_down": dF}
    stages = {}
    for name, us in per.items():
        rec = {"us": round(us, 2)}
        if name in gemm:
            rec["TFLOPs"] = round(gemm[name] / (us * 1e-6) / 1e12, 1)
            rec["frac_peak"] = round(gemm[name] / (us * 1e-6) / PEAK_BF16, 4)
        stages[name] = rec
    bwd_names = [n for n in per if n.startswith("bwd_")]
    bwd_gemm = [n for n in ("bwd_gemm_dh", "bwd_gemm_dx", "bwd_wgrad_w3", "bwd_wgrad_w13") if n in per]
    g_us = sum(per[n] for n in bwd_gemm)
    g_fl = sum(gemm[n] for n in bwd_gemm)
    step_s = (t1 - t0) / steps
    step_rp = (t3 - t2) / steps
    return {"step_ms": round(step_s * 1e3, 3), "tokens_per_s": round(T / step_s, 1),
            "step_ms_with_repack": round(step_rp * 1e3, 3), "tokens_per_s_with_repack": round(T / step_rp, 1),
            "repack_note": "with_repack: every step starts from new parameter versions (as after an optimizer "
                           "update), so the forward and backward packed weights are rebuilt inside the step",
            "backward_us": round(sum(per[n] for n in bwd_names), 1),
            "bwd_expert_gemm_TFLOPs": round(g_fl / (g_us * 1e-6) / 1e12, 1) if g_us else None,
            "bwd_expert_gemm_frac_peak": round(g_fl / (g_us * 1e-6) / PEAK_BF16, 4) if g_us else None,
            "work": "backward expert GEMMs 12*d*F*A_kept FLOP (dh 2, dX 4, dW3 2, dW1|dW2 4)",
            "stages": stages, "steps": steps,
            "note": "forward keeping g/u and the router pre-activation + backward (dy ~ N(0,1) bf16, aux grad 1); "
                    "outside the forward metric's timed region"}


def run_cpu_baseline(wl, tokens):
    """The op-for-op torch-CPU port of the reference path on a bounded sample of
    `tokens` tokens of workload `wl` (one sequence), fp32 (config 5: fp32 with e4m3
    fake quantisation): 1 warm-up, median of 3."""
    import torch
    from kmoe import synth
    from oracle import torch_port as P

    cores = len(os.sched_getaffinity(0))
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)
    wl32 = synth.Workload(wl.name, B=1, S=tokens, d=wl.d, E=wl.E, k=wl.k, F=wl.F, dtype=torch.float32,
                          seed=wl.seed, routing=wl.routing, capacity_factor=wl.capacity_factor,
                          drop_overflow=wl.drop_overflow, zipf_bias=wl.zipf_bias, fp8=wl.fp8, mod=wl.mod,
                          mod_cf=wl.mod_cf)
    t = synth.make_tensors(wl32, "cpu", tokens=tokens)
    x, w_in, w_out, w1, w2, w3 = t["x"], t["w_in"], t["w_out"], t["w1"], t["w2"], t["w3"]
    if wl.mod:
        w1q, w2q, w3q = P.fake_quant_expert_weights(w1, w2, w3)  # static weights: quantised once
        keep = max(1, min(tokens, int(tokens * wl.mod_cf)))
        fn = lambda: P.moe_layer_fp8_mod(x, t["w_mod"], w_in, w_out, w1q, w2q, w3q, wl.k, keep)
        what = (f"MoD keep {keep} of {tokens}, token choice top-{wl.k} on the kept rows, e4m3 fake quantisation "
                f"(float8_e4m3fn casts), oracle/torch_port.py moe_layer_fp8_mod")
    elif wl.routing == "expert_choice":
        fn = lambda: P.moe_layer_ec(x, w_in, w_out, w1, w2, w3, wl.capacity_factor)
        what = (f"expert choice, C = ceil({tokens}*{wl.capacity_factor}/{wl.E}), oracle/torch_port.py moe_layer_ec "
                f"(reference op sequence: gather, repeated-weight bmm, scatter_add_)")
    elif wl.drop_overflow or wl.zipf_bias:
        bias = torch.tensor(synth.zipf_bias(wl.E, wl.seed)) if wl.zipf_bias else None
        x2d = x.reshape(tokens, wl.d)

        def fn():
            logits = torch.nn.functional.linear(torch.nn.functional.silu(torch.nn.functional.linear(x2d, w_in)),
                                                w_out)
            if bias is not None:
                logits = logits + bias
            idx = torch.topk(torch.softmax(logits, dim=-1), wl.k, dim=-1).indices
            cap = int(math.ceil(tokens * wl.k / wl.E * wl.capacity_factor)) if wl.drop_overflow else 0
            return P.moe_tc_routed(x2d, w_in, w_out, w1, w2, w3, idx, capacity=cap, bias=bias, training=True)
        what = (f"Zipf logit bias, capacity factor {wl.capacity_factor} with overflow dropped, "
                f"oracle/torch_port.py moe_tc_routed (reference op sequence: padded bmm experts)")
    else:
        fn = lambda: P.moe_layer_tc(x, w_in, w_out, w1, w2, w3, wl.k, training=True)
        what = "oracle/torch_port.py moe_layer_tc (reference op sequence: padded bmm experts)"
    times = []
    with torch.no_grad():
        for i in range(4):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
    med = statistics.median(times[1:])
    return {"value": round(tokens / med, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{tokens} tokens (one sequence) of {wl.name} (d={wl.d}, E={wl.E}, F={wl.F}), fp32, {what}; "
                      f"median of 3 after 1 warm-up",
            "seconds_per_forward": round(med, 3)}


def library_gemm_reference(wl, a_kept, gu_us):
    """The vendor library's dense bf16 GEMM (torch.mm -> hipBLASLt) of the gate/up shape in
    the same process: (A_kept x d) @ (d x 2F), no grouping and no row gather, K-steps of
    the same size.  A reference for the grouped kernel's rate on this box (same clock and
    power limit), not a replacement: the grouped GEMM has 16 ragged expert groups."""
    import torch
    g = torch.Generator().manual_seed(wl.seed + 400)
    a = (torch.randn(a_kept, wl.d, generator=g) * 0.5).to(torch.bfloat16).to("cuda:0")
    b = (torch.randn(wl.d, 2 * wl.F, generator=g) * 0.02).to(torch.bfloat16).to("cuda:0")
    for _ in range(3):
        torch.mm(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 20
    e0.record()
    for _ in range(n):
        torch.mm(a, b)
    e1.record()
    torch.cuda.synchronize()
    lib_us = e0.elapsed_time(e1) / n * 1e3
    flops = 4.0 * wl.d * wl.F * a_kept
    del a, b
    torch.cuda.empty_cache()
    return {"shape": f"({a_kept} x {wl.d}) @ ({wl.d} x {2 * wl.F}) bf16", "us": round(lib_us, 2),
            "TFLOPs": round(flops / (lib_us * 1e-6) / 1e12, 1), "frac_peak": round(flops / (lib_us * 1e-6) / PEAK_BF16, 4),
            "grouped_gate_up_over_library": round(lib_us / gu_us, 4),
            "note": "torch.mm (hipBLASLt) on the dense gate/up shape, same process, after the timed region; the grouped "
                    "kernel additionally gathers its A rows and handles 16 ragged expert groups"}


def load_traffic(name):
    path = os.path.join(ROOT, "profiles", f"traffic_{name}.json")
    if os.path.exists(path):
        with open(path) as f:
            return json.load(f)
    return None


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on exactly one GPU (no expert parallelism / collectives); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import torch
    from kmoe import synth

    wl = synth.WORKLOADS[args.config]
    if args.calib_copy:
        # reference kernel for PMC byte-counter scaling: reads and writes exactly 512 MiB per launch
        src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.add(src, 1, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes": 512 << 20, "launches": 3}))
        return
    res = run_gpu(args, wl)
    ms = res["elapsed"] / args.steps * 1e3
    tokens_per_s = wl.T * args.steps / res["elapsed"]
    flops_gu = res["work"]["gemm_gate_up"][1]
    peak = PEAK_FP8 if wl.fp8 else PEAK_BF16
    us = res["gemm_us"]  # gate/up launch duration, HIP events inside the timed region
    achieved = flops_gu / (us * 1e-6) / 1e12
    traffic = load_traffic(f"gemm_gate_up_cfg{args.config}")
    out = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "clock_settle": {"ms": args.settle_ms, "extra_untimed_forwards": res["settle"]},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3" if wl.fp8 else "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02^2) weights)",
        "config": {"workload": wl.name, "tokens": wl.T, "d_model": wl.d, "n_experts": wl.E, "top_k": wl.k,
                   "d_ff_expert": wl.F, "routing": wl.routing, "assignments_kept": res["a_kept"]},
        "roofline": {"bound": "mfma", "kernel": "gemm_gate_up", "achieved": round(achieved, 1),
                     "peak": peak / 1e12, "unit": "TFLOP/s", "frac": round(achieved * 1e12 / peak, 4),
                     "traffic": traffic.get("bytes_per_launch") if traffic else None,
                     "traffic_source": (f"profile constant, not measured in this run: profiles/traffic_gemm_gate_up_"
                                        f"cfg{args.config}.json (rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this "
                                        f"kernel, scaled by a plain-copy calibration)") if traffic else None,
                     "work_per_launch": f"4*d*F*A_kept = {flops_gu:.4g} FLOP",
                     "launch_us": round(us, 2), "launch_samples": res["gemm_samples"]},
        "stages": res["stages"],
    }
    gemm_us = res["stages"].get("gemm_gate_up", {}).get("us", 0) + res["stages"].get("gemm_down", {}).get("us", 0)
    if gemm_us:
        tot = res["work"]["gemm_gate_up"][1] + res["work"]["gemm_down"][1]
        out["gemm_frac_peak"] = round(tot / (gemm_us * 1e-6) / peak, 4)
    if "dispatch" in res["stages"]:
        out["dispatch_GBps"] = res["stages"]["dispatch"].get("GBps")
    if res.get("rows_us"):
        # SURVEY definition of the dispatch bytes: read x once, write the kept
        # permuted rows, 8 B of metadata per assignment
        b = wl.T * wl.d * 2 + res["a_kept"] * wl.d * 2 + 8.0 * res["a_all"]
        out["dispatch_rows"] = {"us": round(res["rows_us"], 2), "GBps": round(b / (res["rows_us"] * 1e-6) / 1e9, 1),
                                "frac_hbm": round(b / (res["rows_us"] * 1e-6) / PEAK_HBM, 4),
                                "note": "device time (the host has enqueued the 10 timed calls before the first "
                                        "event fires); materialising dispatch (tables from the router's block histograms + row "
                                        "copy), as the training forward runs it, timed separately; the bf16 inference "
                                        "layer gathers rows inside the gate/up GEMM instead"}
    if "combine" in res["stages"]:
        out["combine_GBps"] = res["stages"]["combine"].get("GBps")
    if res.get("near_ties") is not None:
        out["near_ties"] = res["near_ties"]
    if res.get("training"):
        out["training"] = res["training"]
    if res.get("block"):
        out["ffn_block"] = res["block"]
    if not wl.fp8 and args.library_gemm:
        out["library_gemm"] = library_gemm_reference(wl, res["a_kept"], us)
    if not args.no_configs:
        # the other configurations of BASELINE.json, each with its own timed region
        import argparse as _ap
        sub = _ap.Namespace(**vars(args))
        sub.steps, sub.warmup, sub.stage_steps = args.config_steps, 5, 10
        out["configs"] = {}
        for n in (2, 3, 4, 5):
            if n == args.config:
                continue
            wl_n = synth.WORKLOADS[n]
            out["configs"][f"cfg{n}"] = config_summary(wl_n, run_gpu(sub, wl_n, light=True), sub.steps)
    if not args.no_cpu:
        out["cpu_baseline"] = run_cpu_baseline(synth.WORKLOADS[args.config], args.cpu_tokens)
        if not args.no_configs:
            # the other configurations, each on its own bounded sample (the GPU figures
            # of the 'configs' object are on the full shapes)
            out["cpu_baselines"] = {f"cfg{n}": run_cpu_baseline(synth.WORKLOADS[n], args.cpu_tokens)
                                    for n in (2, 3, 4, 5) if n != args.config}
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

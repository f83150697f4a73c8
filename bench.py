#!/usr/bin/env python3
"""PPO policy minibatch forward + backward throughput on one MI355X (BASELINE.json metric).

One step = one talos_ppo_fwd_bwd_f32 call on the C4 configuration: a minibatch of 4096 gacha
state sequences of 32 tokens through the 2-layer d128 policy (4 heads x 32, RoPE, causal
attention, 4x GELU MLP, last-token actor/critic heads), the clipped PPO loss, and the gradients
of every parameter, all fp32 and resident in HBM before the timed region starts.

Printed (one JSON line): samples/s over the timed steps; the roofline of the dominant kernel
(algorithmic flops or bytes per launch over its average launch time, measured with HIP events
on the stream the kernels run on); and the CPU baseline: the f64 oracle (a C++ restatement of
the reference's Rust autograd) timed on this host's cores on a bounded sample.
"""
import argparse
import glob
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "talos-xii_amd"), os.path.join(ROOT, "oracle")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

import talos_hip as th  # noqa: E402
import workload as wl  # noqa: E402

METRIC = "PPO policy fwd+bwd samples/sec (d128 block, 1 GPU); % MFMA/HBM roofline"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
PEAK_BF16_MFMA_TFLOPS = 2516.6


def ppo_cfg(B, S):
    # batch, seq, in_dim, d_model, n_layers, n_heads, head_dim, ffn_dim, n_actions, causal,
    # activation (GELU), eps, rope_base, clip_eps, value_coef, entropy_coef
    return (B, S, 8, 128, 2, 4, 32, 512, 3, 1, th.ACT_GELU, 1e-5, 10000.0, 0.2, 0.5, 0.01)


def make_inputs(cfg_t, seed=0):
    B, S = cfg_t[0], cfg_t[1]
    cfg = th.PpoCfg(*cfg_t)
    rng = np.random.default_rng(seed)
    p = wl.ppo_params(rng, cfg).astype(np.float32)
    states = wl.gacha_states(rng, B, S).astype(np.float32)
    actions = rng.integers(0, cfg.n_actions, B).astype(np.int32)
    adv = rng.normal(size=B).astype(np.float32)
    ret = rng.normal(size=B).astype(np.float32)
    return cfg, p, states, actions, adv, ret


def aggregate(records):
    agg = {}
    for k, fl, by, ms in records:
        a = agg.setdefault(k, [0, 0.0, 0.0, 0.0])
        a[0] += 1
        a[1] += fl
        a[2] += by
        a[3] += ms
    return agg


def runs_on_bf16_mfma(name):
    """Kernel symbols whose products run on the bf16 matrix cores: the bf16-in GEMMs
    (gemm_f32_kernel<TA, TB, E, true>) and the attention kernels with bf16 in their name."""
    return "bf16" in name or (name.startswith("gemm_f32_kernel") and name.endswith("true>"))


def roofline_of(name, n, flops, bytes_, ms, peak_tflops=None):
    """The roofline of a kernel symbol from its launches: matrix-core bound when its arithmetic
    intensity (algorithmic flops per algorithmic HBM byte) is above the ridge point of the MFMA
    peak it runs on (fp32 157.3 TFLOP/s, or bf16 2.5 PFLOP/s for the bf16-in GEMMs), HBM-bound
    below it. achieved = algorithmic work per launch / average launch time."""
    avg_ms = ms / n
    if peak_tflops is None:
        peak_tflops = PEAK_BF16_MFMA_TFLOPS if runs_on_bf16_mfma(name) else PEAK_FP32_MFMA_TFLOPS
    ridge = peak_tflops * 1e12 / (PEAK_HBM_GBS * 1e9)
    if flops > 0 and (bytes_ <= 0 or flops / bytes_ >= ridge):
        achieved = flops / n / (avg_ms * 1e-3) / 1e12
        return {"bound": "mfma", "achieved": round(achieved, 3), "peak": peak_tflops, "unit": "TFLOP/s",
                "frac": round(achieved / peak_tflops, 4), "intensity_flop_per_byte": round(flops / max(bytes_, 1), 2)}
    achieved = bytes_ / n / (avg_ms * 1e-3) / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "intensity_flop_per_byte": round(flops / max(bytes_, 1), 2)}


def traffic_of(kernel, config="C4"):
    """HBM bytes per launch of the kernel symbol in the given configuration, from the committed
    rocprofv3 --pmc summary of that configuration's run (profiles/traffic.json for C4,
    profiles/traffic_<config>.json for the others), if any."""
    name = "traffic.json" if config == "C4" else f"traffic_{config.lower()}.json"
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    try:
        t = json.load(open(path)).get(kernel)
    except (OSError, ValueError):
        return None
    return round(t["bytes"]) if t else None


def _sized_run(run, n0, n_max, seconds):
    """Calibrates run(n) at n0, then runs it at the n (<= n_max) that takes about `seconds`."""
    t0 = run(n0)
    n = int(max(n0, min(n_max, seconds / max(t0 / n0, 1e-6))))
    return n, run(n)


def cpu_baseline_c3(seconds=6.0):
    """The f64 oracle's C3 block fwd+bwd (a C++ restatement of the reference's Rust autograd) on
    this host's cores, on a bounded number of the 512 sequences, reported as the time of a whole
    C3 step at that rate."""
    import pyoracle
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    pyoracle.set_threads(threads)
    d, H, F = 128, 4, 512
    rng = np.random.default_rng(3)
    p = wl.block_params(rng, d, F, gain_jitter=True)

    def run(b):
        x, G = rng.normal(size=(b, 64, d)), rng.normal(size=(b, 64, d))
        t0 = time.perf_counter()
        pyoracle.block_fwd_bwd(pyoracle.BlockCfg(b, 64, d, H, d // H, F, 1, 0, 1e-6, 1e4), p, x, G)
        return time.perf_counter() - t0

    b, t = _sized_run(run, 2, 512, seconds)
    return {"value": round(t / b * 512 * 1e3, 1), "unit": "ms per C3 step", "cores": threads, "kind": "port",
            "sample": f"{b} of the 512 sequences (seq 64, d128) as one batched f64 graph, the time scaled to 512; "
                      f"C++ restatement of the Rust autograd on {threads} threads"}


def cpu_baseline_c5(seconds=6.0):
    """The f64 oracle's C5 MLA block fwd+bwd on this host's cores on a bounded number of the 64
    sequences, reported as the time of a whole C5 step at that rate."""
    import pyoracle
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    pyoracle.set_threads(threads)
    rng = np.random.default_rng(5)
    p = wl.mla_params(rng, [1, 256, 512, 8, 128, 32, 64, 64, 0])

    def run(b):
        x, G = rng.normal(size=(b, 256, 512)), rng.normal(size=(b, 256, 512))
        t0 = time.perf_counter()
        pyoracle.mla_fwd_bwd([b, 256, 512, 8, 128, 32, 64, 64, 0, 0], 1e-5, 1e4, p, x, G)
        return time.perf_counter() - t0

    b, t = _sized_run(run, 1, 64, seconds)
    return {"value": round(t / b * 64 * 1e3, 1), "unit": "ms per C5 step", "cores": threads, "kind": "port",
            "sample": f"{b} of the 64 sequences (seq 256, d512 MLA) as one batched f64 graph, the time scaled to 64; "
                      f"C++ restatement of the Rust autograd on {threads} threads"}


def cpu_baseline(cfg_t, seconds_budget=20.0):
    """The f64 oracle on this host: reference-faithful per-sample batch-1 graphs (the backbone run
    for the actor and again for the critic, src/ppo.rs:691-757) on a bounded sample, plus the
    batched restatement. Threads: this host's cores, at most 16 (a GPU box's CPU share)."""
    import pyoracle  # prebuilt by __graft_entry__.build(); never compiled from a GPU process
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    pyoracle.set_threads(threads)

    def run(n, per_sample):
        t = ppo_cfg(n, cfg_t[1])
        ocfg = pyoracle.PpoCfg(*t)
        _, p, states, actions, adv, ret = make_inputs(t, seed=1)
        old = np.full(n, -1.1)
        t0 = time.perf_counter()
        if per_sample:
            pyoracle.ppo_fwd_bwd_per_sample(ocfg, p, states, actions, adv, ret, old, True)
        else:
            pyoracle.ppo_fwd_bwd(ocfg, p, states, actions, adv, ret, old)
        return time.perf_counter() - t0

    # calibrate on 4 samples, then size the sample to about half the budget per mode
    t4 = run(4, True)
    n_ps = int(max(8, min(512, 0.5 * seconds_budget / max(t4 / 4, 1e-4))))
    t_ps = run(n_ps, True)
    t16 = run(16, False)
    n_b = int(max(16, min(1024, 0.5 * seconds_budget / max(t16 / 16, 1e-4))))
    t_b = run(n_b, False)
    return {"value": round(n_ps / t_ps, 2), "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": f"{n_ps} samples of the C4 minibatch (seq 32, 2-layer d128), one batch-1 f64 graph per "
                      f"sample with the backbone run for actor and critic as src/ppo.rs:691-757 does; C++ "
                      f"restatement of the Rust autograd on {threads} threads",
            "batched_value": round(n_b / t_b, 2),
            "batched_sample": f"{n_b} samples as one batched f64 graph", "host": host_info()}


def host_info():
    """The host the CPU baseline ran on: CPU model, logical CPUs the OS reports, and the CPUs this
    process may run on."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0))}


def product_names():
    """The marketing names the kernel driver exposes in sysfs for the visible cards (empty where
    there is no such file). Read as files: this process has initialised the GPU, and a child it
    forks must not exec another program, so no rocm-smi."""
    names = []
    for path in sorted(glob.glob("/sys/class/drm/card*/device/product_name")):
        try:
            n = open(path).read().strip()
        except OSError:
            continue
        if n and n not in names:
            names.append(n)
    return names


def device_line():
    """Device 0 as the runtime reports it, with the driver's product name when the runtime gives
    none."""
    info = th.device_info()
    name = info["name"]
    products = product_names()
    if products and name.startswith("AMD GPU with"):
        name = f"{products[0]} {name[name.find('('):]}" if "(" in name else products[0]
    return {"name": name, "cu_count": info["cu_count"], "clock_mhz": info["clock_khz"] // 1000,
            "memory_gib": round(info["total_mem"] / 2 ** 30, 1), "product_names": products}


def optimizer_line(P, dP, steps):
    """The optimizer step on the minibatch's gradients, timed apart from fwd+bwd: Adam over every
    parameter (src/ppo.rs:519-533; 28 B of HBM traffic per parameter) and the DQN variant with
    its global-norm clip (src/dqn.rs:207-239; + one 4 B gradient read for the norm)."""
    n = P.size
    m, v = th.DeviceArray.zeros(n), th.DeviceArray.zeros(n)
    sumsq = th.DeviceArray.zeros(1, np.float64)
    ws = th.DeviceArray.zeros(th.lib().talos_grad_sumsq_workspace_bytes() // 8, np.float64)
    # a copy of the parameters: the timed steps must not move the ones the fwd+bwd line used
    Pc = th.DeviceArray.zeros(n)
    th.call("talos_memcpy_d2d", Pc.ptr, P.ptr, 4 * n, None)
    timer = th.Timer(None)
    res = {"params": n}
    for name, clip in (("adam", False), ("adam_global_norm_clip", True)):
        def one(t):
            if clip:
                th.call("talos_grad_sumsq_f32", n, dP.ptr, 0, sumsq.ptr, ws.ptr, None)
            th.call("talos_adam_step_f32", n, Pc.ptr, dP.ptr, m.ptr, v.ptr, t, 3e-4, 0.9, 0.999, 1e-8,
                    sumsq.ptr if clip else None, 1.0, None)
        for t in range(1, 4):
            one(t)
        th.sync()
        timer.start()
        for t in range(4, 4 + steps):
            one(t)
        us = timer.stop_ms() / steps * 1e3
        nbytes = 28.0 * n + (4.0 * n if clip else 0.0)
        res[name] = {"us_per_step": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
    for a in (m, v, sumsq, ws, Pc):
        a.free()
    return res


def reference_model_line(steps, batch=4096, seq=16):
    """PPO minibatch fwd+bwd of the reference's own ActorCritic (one MLA layer, d 64, ReLU 2x,
    5 actions, no mask) at the trainer's context length 16: the model the reference trains,
    beside the C4 restatement the headline metric is quoted on."""
    cfg_t = (batch, seq, *wl.REFERENCE_ACTOR_CRITIC)
    cfg, p, states, actions, adv, ret = make_inputs(cfg_t, seed=3)
    plan = th.Plan("ppo", cfg)
    P, St = th.DeviceArray.from_numpy(p), th.DeviceArray.from_numpy(states)
    Ac = th.DeviceArray.from_numpy(actions, np.int32)
    Ad, Re = th.DeviceArray.from_numpy(adv), th.DeviceArray.from_numpy(ret)
    Ol = th.DeviceArray.from_numpy(np.full(batch, -1.6, np.float32))
    loss, dP = th.DeviceArray.zeros(1), th.DeviceArray.zeros(p.size)

    def step():
        th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dP.ptr, None)

    for _ in range(3):
        step()
    th.sync()
    timer = th.Timer(None)
    timer.start()
    for _ in range(steps):
        step()
    ms = timer.stop_ms() / steps
    plan.destroy()
    for a in (P, St, Ac, Ad, Re, Ol, loss, dP):
        a.free()
    return {"workload": f"reference ActorCritic minibatch fwd+bwd, {batch} samples x seq {seq}",
            "samples_per_s": round(batch / (ms * 1e-3), 1), "ms_per_step": round(ms, 4), "params": int(p.size)}


def rollout_line(steps, n_envs=4096, context_len=16, cpu=True):
    """Rollout inference with the KV cache on the reference's own ActorCritic (one MLA layer,
    d 64; ActorCritic::new, src/ppo.rs:254-258): one token for each of n_envs environments per
    step, the cache window of ppo_context_len 16 (data/config.json:53-54), actions drawn
    (step_inference_cached, src/ppo.rs:391-433). The caches are filled to the window before the
    timed steps. The CPU baseline is the oracle's f64 restatement of forward_inference_step on
    one thread for a bounded number of environment-steps (the reference decodes each simulation
    on its own thread)."""
    cfg_t = (1, context_len, *wl.REFERENCE_ACTOR_CRITIC)
    cfg = th.PpoCfg(*cfg_t)
    rng = np.random.default_rng(5)
    p = wl.ppo_params(rng, cfg).astype(np.float32)
    dec = th.Decoder(cfg, n_envs, context_len, 256)
    P = th.DeviceArray.from_numpy(p)
    toks = th.DeviceArray.from_numpy(wl.gacha_states(rng, n_envs, 1)[:, 0].astype(np.float32))
    u = th.DeviceArray.from_numpy(rng.random(n_envs).astype(np.float32))
    lg = th.DeviceArray.zeros((n_envs, cfg.n_actions))
    vl, lp = th.DeviceArray.zeros(n_envs), th.DeviceArray.zeros(n_envs)
    act = th.DeviceArray.zeros(n_envs, np.int32)
    pos = [th.DeviceArray.from_numpy(np.full(n_envs, t, np.int32), np.int32) for t in range(context_len + steps)]

    def one(t):
        dec.step(n_envs, P, toks, pos[t], None, u, lg, vl, act, lp)

    for t in range(context_len):
        one(t)
    th.sync()
    timer = th.Timer(None)
    timer.start()
    for t in range(context_len, context_len + steps):
        one(t)
    ms = timer.stop_ms() / steps
    res = {"workload": f"reference ActorCritic (1 MLA layer, d 64), {n_envs} environments x 1 token per step, "
                       f"cache window {context_len}, caches full; logits, value, action and log-prob per token",
           "tokens_per_s": round(n_envs / (ms * 1e-3), 1), "us_per_step": round(ms * 1e3, 2)}
    if cpu:
        import pyoracle
        ocfg = pyoracle.PpoCfg(*cfg_t)
        od = pyoracle.Decoder(ocfg, p.astype(np.float64), 256, 1)
        x = wl.gacha_states(rng, 1, 1)[0, 0]
        for t in range(context_len):
            od.step(0, x, t)
            od.prune(0, context_len)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 2.0:
            od.step(0, x, context_len + n)
            od.prune(0, context_len)
            n += 1
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": round(n / dt, 1), "unit": "tokens/s", "cores": 1, "kind": "port",
                               "sample": f"{n} environment-steps of the f64 restatement of forward_inference_step "
                                         f"+ prune_kv_cache, window {context_len}, one thread"}
    for a in [P, toks, u, lg, vl, lp, act] + pos:
        a.free()
    dec.destroy()
    return res


def dominant_roofline(plan, step, steps, config):
    """One profiled step for the per-kernel table, then `steps` steps with the launches of the
    kernel symbol that took the most time bracketed by HIP events on their stream: its roofline,
    with the counter-measured traffic of that symbol in this configuration's profile."""
    plan.profile(True)
    step()
    th.sync()
    agg = aggregate(plan.profile_records())
    plan.profile(False)
    dominant = max(agg, key=lambda k: agg[k][3])
    plan.profile(True, dominant)
    for _ in range(steps):
        step()
    th.sync()
    n, fl, by, ms = aggregate(plan.profile_records())[dominant]
    plan.profile(False)
    roof = roofline_of(dominant, n, fl, by, ms)
    roof.update({"kernel": dominant, "launches_per_step": n // steps, "avg_launch_us": round(ms / n * 1e3, 2),
                 "traffic": traffic_of(dominant, config),
                 "algorithmic_per_launch": {"flops": fl / n, "bytes": by / n}})
    total = sum(a[3] for a in agg.values())
    kernels = {k: {"launches": v[0], "ms": round(v[3], 4), "pct": round(100 * v[3] / total, 1)}
               for k, v in sorted(agg.items(), key=lambda kv: -kv[1][3])}
    return roof, kernels


def timed(step, steps, warmup):
    for _ in range(warmup):
        step()
    th.sync()
    timer = th.Timer(None)
    timer.start()
    for _ in range(steps):
        step()
    return timer.stop_ms() / steps


def c3_line(steps, warmup):
    """C3: one pre-norm block forward + backward at batch 512, seq 64, d_model 128, 4 heads x 32,
    RoPE, causal attention, 4x GELU MLP, loss = sum(out * G): talos_block_fwd_bwd_f32 on
    device-resident inputs. Work: the forward's four d x d products and two MLP products over the
    32768 tokens plus causal attention, the backward twice that (3 x 13.43 = 40.3 GFLOP)."""
    B, S, d, H, F = 512, 64, 128, 4, 512
    cfg = th.BlockCfg(B, S, d, H, d // H, F, 1, th.ACT_GELU, 1e-6, 10000.0)
    rng = np.random.default_rng(3)
    p = wl.block_params(rng, d, F, gain_jitter=True).astype(np.float32)
    plan = th.Plan("block", cfg)
    P = th.DeviceArray.from_numpy(p)
    X = th.DeviceArray.from_numpy(rng.normal(size=(B, S, d)).astype(np.float32))
    G = th.DeviceArray.from_numpy(rng.normal(size=(B, S, d)).astype(np.float32))
    out, dP, dX = th.DeviceArray.zeros((B, S, d)), th.DeviceArray.zeros(p.size), th.DeviceArray.zeros((B, S, d))

    def step():
        th.call("talos_block_fwd_bwd_f32", plan.h, P.ptr, X.ptr, G.ptr, out.ptr, dP.ptr, dX.ptr, None)

    ms = timed(step, steps, warmup)
    roof, kernels = dominant_roofline(plan, step, steps, "C3")
    M, hd = B * S, d // H
    flops = 3.0 * (4 * 2 * M * d * d + 2 * 2 * M * d * F + 2 * 2 * B * H * hd * S * (S + 1) / 2)
    plan.destroy()
    tf = flops / (ms * 1e-3) / 1e12
    return {"metric": "C3 pre-norm block fwd+bwd ms/step (B512 S64 d128, 1 GPU); % fp32 MFMA roofline",
            "value": round(ms, 4), "unit": "ms", "higher_is_better": False, "steps": steps, "warmup": warmup,
            "dtype": "fp32", "data": "synthetic",
            "config": {"workload": "C3: one pre-norm transformer block fwd+bwd, batch 512 x seq 64, d_model 128, "
                                   "4 heads x 32, RoPE, causal attention, 4x GELU MLP, loss sum(out * G)"},
            "step": {"algorithmic_gflop": round(flops / 1e9, 2), "tflops": round(tf, 2),
                     "frac_fp32_mfma_peak": round(tf / PEAK_FP32_MFMA_TFLOPS, 4), "target_ms": 0.51},
            "roofline": roof, "kernels": kernels, "device": device_line()}


def c5_line(steps, warmup, precision):
    """C5: the MLA block forward + backward at batch 64, seq 256, d_model 512, 8 heads, KV latent
    128, decoupled RoPE 32, head and value dims 64 (talos_mla_fwd_bwd_f32), fp32 or with the
    bf16-in / fp32-accumulate GEMMs. Work: the seven projections over 16384 tokens (32.21 GFLOP)
    and full attention over 256 x 256 pairs per head with q/k width 96 and v width 64 (10.74
    GFLOP), the backward twice that."""
    ci = [64, 256, 512, 8, 128, 32, 64, 64, 0]
    B, S, d, H, L, r, hd, vd, causal = ci
    cfg = th.MlaCfg(B, S, d, H, L, r, hd, vd, causal, precision, 1e-5, 10000.0)
    rng = np.random.default_rng(5)
    p = wl.mla_params(rng, ci).astype(np.float32)
    plan = th.Plan("mla", cfg)
    P = th.DeviceArray.from_numpy(p)
    X = th.DeviceArray.from_numpy(rng.normal(size=(B, S, d)).astype(np.float32))
    G = th.DeviceArray.from_numpy(rng.normal(size=(B, S, d)).astype(np.float32))
    out, dP, dX = th.DeviceArray.zeros((B, S, d)), th.DeviceArray.zeros(p.size), th.DeviceArray.zeros((B, S, d))

    def step():
        th.call("talos_mla_fwd_bwd_f32", plan.h, P.ptr, X.ptr, G.ptr, out.ptr, dP.ptr, dX.ptr, None)

    ms = timed(step, steps, warmup)
    bf = precision == th.PREC_BF16
    roof, kernels = dominant_roofline(plan, step, steps, "C5")
    M = B * S
    gemm = 2.0 * M * (d * L + L * H * hd + L * H * vd + d * H * hd + 2 * d * H * r + H * vd * d)
    attn = 2.0 * B * H * S * S * ((hd + r) + vd)
    flops = 3.0 * (gemm + attn)
    plan.destroy()
    tf = flops / (ms * 1e-3) / 1e12
    peak = PEAK_BF16_MFMA_TFLOPS if bf else PEAK_FP32_MFMA_TFLOPS
    return {"metric": f"C5 MLA block fwd+bwd ms/step (B64 S256 d512, {'bf16-in/fp32-acc' if bf else 'fp32'}, 1 GPU)",
            "value": round(ms, 4), "unit": "ms", "higher_is_better": False, "steps": steps, "warmup": warmup,
            "dtype": "bf16-in/fp32-acc" if bf else "fp32", "data": "synthetic",
            "config": {"workload": "C5: MLA attention block fwd+bwd, batch 64 x seq 256, d_model 512, 8 heads, "
                                   "KV latent 128, decoupled RoPE 32, head / value dims 64, RMSNorm, no mask"},
            "step": {"algorithmic_gflop": round(flops / 1e9, 2), "tflops": round(tf, 2),
                     "frac_mfma_peak": round(tf / peak, 4), "mfma_peak_tflops": peak},
            "roofline": roof, "kernels": kernels, "device": device_line()}


# the kernel symbols one call of each C2 op launches (their counter traffic is summed)
C2_KERNELS = {"rmsnorm_bwd": ["rmsnorm_bwd_kernel<1>", "reduce_parts_kernel"],
              "softmax_causal_bwd": ["softmax_bwd_rows_kernel<1>"], "rope_bwd": ["rope4_kernel"]}


def c2_line(steps):
    """C2: the standalone row-op backward kernels on [4096, 256] fp32 rows: RMSNorm backward (eps
    1e-6, gain U(0.9,1.1), with the gain gradient), causal softmax backward (row r is query r mod
    256), and RoPE backward on [64 sequences x 64 positions, 4 heads, 64] (base 1e4). Each runs on
    rotating buffer sets of more than 300 MB in all, so the 256 MB Infinity Cache cannot hold the
    operands between launches. `steps` launches over the sets are captured into one HIP graph (the
    entries in their asynchronous mode, a caller-owned workspace bound, so no launch allocates);
    the time per launch is the HIP-event time of a graph replay divided by `steps` (median of three
    replays), i.e. GPU time with the host's per-call cost taken out. Beside each op, the runtime's
    own device-to-device copy (hipMemcpyAsync) of the same bytes over the same rotation is timed the
    same way (one 4 MiB tensor, 8 MiB moved): the floor a launch of that size reaches on this GPU.
    Algorithmic bytes per launch:
    RMSNorm x, dy read and dx written (3 x 4 MiB) plus rstd and the gain read and its gradient
    written; softmax y and dy read on the kept (unmasked) entries only and dx written densely; RoPE
    dy read and dx written plus the cos / sin table."""
    R, C = 4096, 256
    rng = np.random.default_rng(2)
    ws = th.DeviceArray.zeros(1 << 20)
    th.call("talos_workspace_bind", ws.ptr, 4 << 20)
    stream = th.stream_create()
    timer = th.Timer(stream)
    H = th.hip_runtime()
    res = {}

    def per_launch_us(sets, launch):
        for i in range(len(sets)):
            launch(sets[i])
        th.call("talos_stream_sync", stream)
        g = th.Graph(stream, lambda: [launch(sets[i % len(sets)]) for i in range(steps)])
        g.launch()
        th.call("talos_stream_sync", stream)
        t = []
        for _ in range(3):
            timer.start()
            g.launch()
            t.append(timer.stop_ms() / steps * 1e3)
        return sorted(t)[1]

    def measure(name, nbytes, sets, launch, copy_bytes, kernels):
        us = per_launch_us(sets, launch)
        # the runtime's copy of copy_bytes from the first buffer of a set into its output buffer
        cus = per_launch_us(sets, lambda b: th._hip_check(
            H.hipMemcpyAsync(b[-1].ptr, b[0].ptr, copy_bytes, 3, stream), "hipMemcpyAsync"))
        gbs = nbytes / (us * 1e-6) / 1e9
        traffic = [traffic_of(k, "C2") for k in kernels]
        res[name] = {"us_per_launch": round(us, 3), "algorithmic_bytes": int(nbytes), "GB/s": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4), "buffer_sets": len(sets),
                     "rotated_mb": round(len(sets) * sum(a.nbytes for a in sets[0]) / 1e6, 1),
                     "copy_floor_us": round(cus, 3), "copy_floor_bytes": int(2 * copy_bytes),
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                  "frac": round(gbs / PEAK_HBM_GBS, 4), "kernels": kernels,
                                  "traffic": sum(traffic) if None not in traffic else None}}

    try:
        # RMSNorm backward
        x = rng.normal(size=(R, C)).astype(np.float32)
        w = rng.uniform(0.9, 1.1, C).astype(np.float32)
        rstd = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(1) + 1e-6)).astype(np.float32)
        sets = []
        for _ in range(25):
            sets.append([th.DeviceArray.from_numpy(x), th.DeviceArray.from_numpy(rng.normal(size=(R, C))),
                         th.DeviceArray.from_numpy(rstd), th.DeviceArray.from_numpy(w), th.DeviceArray.zeros(C),
                         th.DeviceArray.zeros((R, C))])
        measure("rmsnorm_bwd", 3 * R * C * 4 + R * 4 + 2 * C * 4, sets,
                lambda b: th.call("talos_rmsnorm_bwd_f32", R, C, b[0].ptr, b[3].ptr, b[2].ptr, b[1].ptr, 0.0, b[5].ptr,
                                  0.0, b[4].ptr, stream), R * C * 4, C2_KERNELS["rmsnorm_bwd"])
        for b in sets:
            for a in b:
                a.free()
        # causal softmax backward
        sm = np.exp(rng.normal(size=(R, C)))
        q = np.arange(R) % C
        sm[np.arange(C)[None, :] > q[:, None]] = 0.0
        sm = (sm / sm.sum(1, keepdims=True)).astype(np.float32)
        sets = [[th.DeviceArray.from_numpy(sm), th.DeviceArray.from_numpy(rng.normal(size=(R, C))),
                 th.DeviceArray.zeros((R, C))] for _ in range(25)]
        kept = int(np.sum(q + 1))
        measure("softmax_causal_bwd", 2 * kept * 4 + R * C * 4, sets,
                lambda b: th.call("talos_softmax_bwd_f32", R, C, 1, b[0].ptr, b[1].ptr, 0.0, b[2].ptr, stream),
                R * C * 4, C2_KERNELS["softmax_causal_bwd"])
        for b in sets:
            for a in b:
                a.free()
        # RoPE backward on [64, 64, 4, 64]
        sets = [[th.DeviceArray.from_numpy(rng.normal(size=(64, 64, 4, 64))), th.DeviceArray.zeros((64, 64, 4, 64))]
                for _ in range(37)]
        measure("rope_bwd", 2 * R * C * 4 + 2 * 64 * 32 * 4, sets,
                lambda b: th.call("talos_rope_bwd_f32", 64, 64, 4, 64, 0, 10000.0, b[0].ptr, 0.0, b[1].ptr, stream),
                R * C * 4, C2_KERNELS["rope_bwd"])
        for b in sets:
            for a in b:
                a.free()
    finally:
        th.call("talos_workspace_bind", None, 0)
        ws.free()
        th.stream_destroy(stream)
    return {"metric": "C2 row-op backward HBM GB/s ([4096,256] RMSNorm / causal softmax, RoPE [4096,4,64]; 1 GPU)",
            "value": res, "unit": "GB/s", "higher_is_better": True, "steps": steps, "dtype": "fp32",
            "data": "synthetic",
            "config": {"workload": "C2: standalone RMSNorm backward (eps 1e-6, gain U(0.9,1.1)) and causal softmax "
                                   "backward on [4096,256], RoPE backward on [4096 = 64 x 64 positions, 4, 64]"},
            "target_us": {"rmsnorm_bwd": 2.62, "softmax_causal_bwd": 1.75, "rope_bwd": 1.75},
            "device": device_line()}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=4096)
    ap.add_argument("--seq", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave the C2 / C3 / C5 results out of the default line")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--profile-table", action="store_true", help="print the per-kernel table to stderr")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the C4 line (no optimizer, reference-model or rollout lines): the command to run "
                         "under rocprofv3, so that its per-kernel averages cover the headline step alone")
    ap.add_argument("--rollout-only", action="store_true",
                    help="only the rollout line (its JSON object alone): the command to run under rocprofv3 for "
                         "the rollout kernel's averages")
    ap.add_argument("--config", default="C4", choices=["C4", "C2", "C3", "C5", "all"],
                    help="C4 (default): the headline PPO minibatch line; C2 / C3 / C5: the line of that "
                         "configuration instead (C5 prints fp32 and bf16 lines); all: every line, C4 first")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB device-to-device 5 times: the known-size "
                         "copy that scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "The minibatch would shard over samples, each GPU running this step on its share, with one "
              "all-reduce of the parameter gradients.",
              file=sys.stderr)
        sys.exit(2)
    rank = int(os.environ.get("RANK", "0"))
    # the library's entries are synchronous by default (the reference's semantics); a training
    # loop enqueues its steps back to back, so the timed loops run in the asynchronous mode and
    # wait once, at the end of the timed region
    th.call("talos_set_async", 1)
    if args.rollout_only:
        print(json.dumps({"rollout": rollout_line(args.steps, cpu=False)}))
        return
    if args.config == "all":
        args.no_configs = True  # each configuration prints its own line
    if args.config in ("C4", "all"):
        main_c4(args, rank)
    elif args.copy_calibration_mb > 0:
        print(json.dumps({"copy_calibration_bytes": copy_calibration(args.copy_calibration_mb)}), flush=True)
    if args.config in ("C2", "all"):
        print(json.dumps(c2_line(max(args.steps, 200))), flush=True)
    cpu = rank == 0 and not args.no_cpu_baseline
    if args.config in ("C3", "all"):
        line = c3_line(args.steps, args.warmup)
        if cpu:
            line["cpu_baseline"] = cpu_baseline_c3()
        print(json.dumps(line), flush=True)
    if args.config in ("C5", "all"):
        for prec in (th.PREC_FP32, th.PREC_BF16):
            line = c5_line(args.steps, args.warmup, prec)
            if cpu and prec == th.PREC_FP32:
                line["cpu_baseline"] = cpu_baseline_c5()
            print(json.dumps(line), flush=True)


def other_configs(args, rank):
    """The other configurations of BASELINE.json, measured in the default run beside the headline
    line: C2's row-op backward kernels, the C3 block and the C5 MLA block in fp32 and bf16-in, each
    with its roofline (the C2 ops per op; C3 and C5 of their dominant kernel) and, on rank 0, the
    f64 oracle's time for the same work on this host (C3, C5)."""
    cpu = rank == 0 and not args.no_cpu_baseline

    def trim(line, top=6):
        out = {k: v for k, v in line.items() if k not in ("kernels", "device", "steps", "warmup", "data")}
        out["top_kernels"] = dict(list(line["kernels"].items())[:top])
        return out

    res = {}
    c2 = c2_line(max(args.steps, 200))
    res["C2"] = {k: c2[k] for k in ("metric", "value", "unit", "target_us")}
    res["C3"] = trim(c3_line(args.steps, args.warmup))
    if cpu:
        res["C3"]["cpu_baseline"] = cpu_baseline_c3()
    res["C5_fp32"] = trim(c5_line(args.steps, args.warmup, th.PREC_FP32))
    res["C5_bf16"] = trim(c5_line(args.steps, args.warmup, th.PREC_BF16))
    if cpu:
        res["C5_fp32"]["cpu_baseline"] = cpu_baseline_c5()
    return res


def main_c4(args, rank):
    """The headline line: the C4 PPO minibatch (and, unless --headline-only, the optimizer,
    reference-model and rollout side lines)."""
    cfg_t = ppo_cfg(args.batch, args.seq)
    cfg, p, states, actions, adv, ret = make_inputs(cfg_t)
    B = cfg.batch
    plan = th.Plan("ppo", cfg)
    P, St = th.DeviceArray.from_numpy(p), th.DeviceArray.from_numpy(states)
    Ac = th.DeviceArray.from_numpy(actions, np.int32)
    Ad, Re = th.DeviceArray.from_numpy(adv), th.DeviceArray.from_numpy(ret)
    # old log-probs: the initial policy's (ratio = 1 on the first epoch, as in a PPO update)
    lg, vl = th.DeviceArray.zeros((B, cfg.n_actions)), th.DeviceArray.zeros(B)
    th.call("talos_ppo_forward_f32", plan.h, P.ptr, St.ptr, lg.ptr, vl.ptr, None)
    old = wl.log_softmax(lg.numpy().astype(np.float64))[np.arange(B), actions].astype(np.float32)
    Ol = th.DeviceArray.from_numpy(old)
    loss, dP = th.DeviceArray.zeros(1), th.DeviceArray.zeros(p.size)

    def step():
        th.call("talos_ppo_fwd_bwd_f32", plan.h, P.ptr, St.ptr, Ac.ptr, Ad.ptr, Re.ptr, Ol.ptr, loss.ptr, dP.ptr, None)

    for _ in range(args.warmup):
        step()
    th.sync()
    assert np.isfinite(loss.numpy()[0]), "non-finite loss"

    # 1) per-kernel breakdown of one step (all launches event-bracketed)
    plan.profile(True)
    step()
    th.sync()
    agg = aggregate(plan.profile_records())
    plan.profile(False)
    dominant = max(agg, key=lambda k: agg[k][3])

    # 2) the timed region: K steps, synchronised on both sides
    timer = th.Timer(None)
    th.sync()
    timer.start()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ms_total = timer.stop_ms()
    wall = time.perf_counter() - t0
    ms_step = ms_total / args.steps
    value = B * args.steps / (ms_total * 1e-3)

    # 3) the same K steps again with the dominant kernel's launches event-bracketed
    plan.profile(True, dominant)
    for _ in range(args.steps):
        step()
    th.sync()
    dom = aggregate(plan.profile_records()).get(dominant)
    plan.profile(False)
    n, fl, by, ms = dom
    roof = roofline_of(dominant, n, fl, by, ms)
    roof["kernel"] = dominant
    roof["launches_per_step"] = n // args.steps
    roof["avg_launch_us"] = round(ms / n * 1e3, 2)
    roof["traffic"] = traffic_of(dominant)
    roof["algorithmic_per_launch"] = {"flops": fl / n, "bytes": by / n}

    # live work (what the loss depends on; the plan skips the last layer's dead rows) and the
    # reference's whole graph
    shape = (B, cfg.seq, cfg.in_dim, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.ffn_dim, cfg.n_actions)
    step_flops = wl.ppo_step_flops(*shape)
    graph_flops = wl.ppo_step_flops(*shape, live=False)
    exec_flops = wl.ppo_step_executed_flops(*shape)
    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "samples/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp32", "data": "synthetic",
        "config": {"workload": "C4: PPO policy minibatch fwd+bwd, 4096 samples x seq 32 gacha states (8 features), "
                               "2-layer pre-norm d128, 4 heads x 32, RoPE, causal attention, 4x GELU MLP, 3 actions",
                   "batch": B, "seq": cfg.seq, "d_model": cfg.d_model, "n_layers": cfg.n_layers,
                   "n_heads": cfg.n_heads, "ffn_dim": cfg.ffn_dim, "n_actions": cfg.n_actions},
        "roofline": roof,
        "step": {"algorithmic_gflop": round(step_flops / 1e9, 2),
                 "reference_graph_gflop": round(graph_flops / 1e9, 2),
                 "executed_gflop": round(exec_flops / 1e9, 2),
                 "tflops": round(step_flops / (ms_step * 1e-3) / 1e12, 2),
                 "frac_fp32_mfma_peak": round(step_flops / (ms_step * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
                 "executed_tflops": round(exec_flops / (ms_step * 1e-3) / 1e12, 2),
                 "executed_frac_fp32_mfma_peak": round(exec_flops / (ms_step * 1e-3) / 1e12 / PEAK_FP32_MFMA_TFLOPS,
                                                       4),
                 "wall_ms_per_step": round(wall * 1e3 / args.steps, 4)},
        "kernels": {k: {"launches": v[0], "ms": round(v[3], 4), "pct": round(100 * v[3] / sum(a[3] for a in agg.values()), 1)}
                    for k, v in sorted(agg.items(), key=lambda kv: -kv[1][3])},
        "device": device_line(),
    }
    if not args.headline_only:
        out["optimizer"] = optimizer_line(P, dP, args.steps)
        out["reference_model"] = reference_model_line(args.steps)
        out["rollout"] = rollout_line(args.steps, cpu=rank == 0 and not args.no_cpu_baseline)
    if not args.headline_only and not args.no_configs:
        out["configs"] = other_configs(args, rank)
    if args.profile_table:
        for k, v in sorted(agg.items(), key=lambda kv: -kv[1][3]):
            print(f"{k:40s} n={v[0]:3d} {v[3]:8.3f} ms  {v[1] / max(v[3], 1e-9) / 1e9:8.2f} TFLOP/s "
                  f"{v[2] / max(v[3], 1e-9) / 1e6:8.1f} GB/s", file=sys.stderr)
    if rank == 0 and not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(cfg_t, args.cpu_seconds)
    elif rank == 0:
        out["cpu_baseline"] = None
    plan.destroy()
    if args.copy_calibration_mb > 0:
        out["copy_calibration_bytes"] = copy_calibration(args.copy_calibration_mb)
    if rank == 0:
        print(json.dumps(out))


def copy_calibration(mb):
    """Five device-to-device copies of mb MiB: the known-size copy that scales rocprofv3
    FETCH_SIZE / WRITE_SIZE counters to bytes (talos-xii_amd/prof_summary.py)."""
    nbytes = mb << 20
    src, dst = th.DeviceArray.zeros(nbytes // 4), th.DeviceArray.zeros(nbytes // 4)
    for _ in range(5):
        th.call("talos_memcpy_d2d", dst.ptr, src.ptr, nbytes, None)
    th.sync()
    src.free()
    dst.free()
    return nbytes


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Benchmark of the MTP draft+verify decode step's hot path on one MI355X.

Headline (`value`): BASELINE config 2 -- one routed-expert block at
DeepSeek-V3 expert shape (hidden 7168, inter 2048, 256 int4 experts, top-8 of
N(0,1) router logits, M=1 token row) -- in achieved algorithmic HBM GB/s.
A step = route (sigmoid, group limit, top-k) + gate/up + SiLU*mul + down +
choice-order combine, with fresh routing logits every step over the 5.6 GB
expert pool (so the 256 MB MALL does not hold the working set).  Inputs are
resident in HBM before the timed region.  The K timed steps are queued
behind a GPU-side wait (outside the timed region) so the events bracket the
GPU work, not Python's launch rate; the host-paced figure (each step
launched as the host reaches it) is reported beside it.

Also reported: M=2/4 and int8 variants, the roofline of the dominant kernel
(fused gate/up, timed with HIP events on the stream it runs on), the
reference CPU path on the host's cores (`cpu_baseline`), and MTP decode
tok/s at batch 1 for config 1 (tiny) and config 4 (DeepSeek-V3 width,
4 layers).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ------------------------------------------------------------- config 2 --
def build_experts(U, ctx, torch, n, hidden, inter, fmt, seed):
    """n experts of uniform codes and |N(0,0.02)|/qmax per-row scales, made on device."""
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    qmax = 7.0 if fmt == U.INT4 else 127.0
    tbl = U.ExpertTable(ctx, n, hidden, inter)

    def qt(o, i):
        if fmt == U.INT4:
            p = torch.randint(0, 256, (o, (i + 1) // 2), dtype=torch.uint8, device="cuda:0", generator=g)
        else:
            p = torch.randint(-127, 128, (o, i), dtype=torch.int8, device="cuda:0", generator=g)
        s = (torch.randn(o, device="cuda:0", generator=g).abs() * 0.02 / qmax).float()
        return U.QTensor(ctx, fmt, p, s, o, i)

    for e in range(n):
        tbl.set(e, qt(inter, hidden), qt(inter, hidden), qt(hidden, inter))
    torch.cuda.synchronize()
    return tbl


_CYCLES_PER_MS = None


def gpu_wait(torch, ms: float) -> None:
    """Hold the current stream for about `ms` (a spin kernel), so launches
    queued behind it start back to back."""
    global _CYCLES_PER_MS
    if _CYCLES_PER_MS is None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1_000_000)  # warm
        e0.record()
        torch.cuda._sleep(4_000_000)
        e1.record()
        torch.cuda.synchronize()
        _CYCLES_PER_MS = 4_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(ms * _CYCLES_PER_MS))


def expert_block_bench(U, ctx, torch, tbl, cfg, M, steps, warmup, fmt_bits, seed, fused=True,
                       bf16x=False):
    """Time `steps` expert-block passes; returns dict with GB/s and kernel times.
    bf16x: the activations x are bf16 (the _bf16 entry points)."""
    from undertow_amd.configs import expert_bytes, gate_up_bytes
    E, H, I, k = cfg["n_experts"], cfg["hidden"], cfg["inter"], cfg["top_k"]
    g = torch.Generator(device="cuda:0")
    g.manual_seed(seed)
    n = steps + warmup
    logits = torch.randn(n, M, E, device="cuda:0", generator=g)
    x = torch.randn(M, H, device="cuda:0", generator=g)
    if bf16x:
        x = x.to(torch.bfloat16)
    xb = x.element_size()
    ids_all = torch.empty(n, M, k, dtype=torch.int32, device="cuda:0")
    w_all = torch.empty(n, M, k, dtype=torch.float32, device="cuda:0")
    out = torch.empty(M, H, device="cuda:0")
    lib = U.lib()

    def step(i):
        if not fused:
            ctx.check(lib.ut_route(ctx.handle, logits[i].data_ptr(), None, M, E, k,
                                   cfg["n_group"], cfg["topk_group"], cfg["norm_topk_prob"],
                                   cfg["routed_scaling_factor"], ids_all[i].data_ptr(),
                                   w_all[i].data_ptr()))
            fn = lib.ut_moe_experts_bf16 if bf16x else lib.ut_moe_experts
            ctx.check(fn(ctx.handle, tbl._h, ids_all[i].data_ptr(), w_all[i].data_ptr(), M, k,
                         x.data_ptr(), out.data_ptr()))
            return
        # route + routed experts (moe_forward's body, model.rs:210-281) in
        # one call; at one row the routing runs inside the gate/up launch
        fn = lib.ut_moe_route_experts_bf16 if bf16x else lib.ut_moe_route_experts
        ctx.check(fn(ctx.handle, tbl._h, logits[i].data_ptr(), None, M, k, cfg["n_group"],
                     cfg["topk_group"], cfg["norm_topk_prob"], cfg["routed_scaling_factor"],
                     x.data_ptr(), out.data_ptr(), ids_all[i].data_ptr(), w_all[i].data_ptr()))

    for i in range(warmup):
        step(i)
    ctx.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ts = torch.cuda.Event(enable_timing=True)
    # host-paced: each step launched as the host reaches it
    t0.record()
    h0 = time.perf_counter()
    for i in range(warmup, n):
        step(i)
    host_ms = (time.perf_counter() - h0) * 1e3
    t1.record()
    ctx.synchronize()
    host_paced_ms = t0.elapsed_time(t1) / steps
    # queued: a GPU-side wait (outside the timed region, three times the
    # host's enqueueing time) lets the host enqueue all `steps` launches
    # first, so the events bracket the GPU work alone; the wait is checked to
    # have outlasted the enqueueing
    wait_for = max(5.0, 3.0 * host_ms)
    ts.record()
    gpu_wait(torch, wait_for)
    t0.record()
    h0 = time.perf_counter()
    for i in range(warmup, n):
        step(i)
    enqueue_ms = (time.perf_counter() - h0) * 1e3
    t1.record()
    ctx.synchronize()
    wait_ms = ts.elapsed_time(t0)
    ms = t0.elapsed_time(t1) / steps
    if enqueue_ms >= wait_ms:  # the GPU caught up with the host: host-paced after all
        log(f"queue wait {wait_ms:.2f} ms shorter than enqueueing {enqueue_ms:.2f} ms")
        ms = max(ms, host_paced_ms)
    ids = ids_all[warmup:].cpu().numpy()
    uniq = [len(np.unique(ids[s])) for s in range(steps)]
    u_mean = float(np.mean(uniq))
    bytes_step = u_mean * expert_bytes(H, I, fmt_bits) + M * H * (xb + 4)
    # per-kernel durations (events around each launch) in a second pass,
    # queued behind a GPU-side wait like the timed region
    ctx.enable_timing(True)
    gpu_wait(torch, wait_for * 3.0)  # events make enqueueing slower
    for i in range(warmup, n):
        step(i)
    ctx.synchronize()
    sfx = "int4" if fmt_bits == 4 else "int8"
    gl, gms = ctx.kernel_time(f"moe_gate_up_{sfx}")
    dl, dms = ctx.kernel_time(f"moe_down_{sfx}")
    tl, tms = ctx.kernel_time("")
    ctx.enable_timing(False)
    gu_bytes = u_mean * gate_up_bytes(H, I, fmt_bits) + M * H * xb
    dn_bytes = u_mean * (H * ((I * fmt_bits + 7) // 8) + H * 4) + u_mean * M * I * 4

    def rate(nbytes, launches, total_ms):
        return nbytes / (total_ms / launches * 1e-3) / 1e9 if launches else None

    r = {
        "M": M, "x_dtype": "bf16" if bf16x else "f32", "unique_experts_mean": u_mean, "ms_per_step": ms,
        "host_paced_ms_per_step": host_paced_ms,
        "bytes_per_step": bytes_step, "gbs": bytes_step / (ms * 1e-3) / 1e9,
        "kernels_us_per_step": tms / steps * 1e3,
        "launches_per_step": tl / steps,
    }
    if gl:
        r.update({"gate_up_us": gms / gl * 1e3, "gate_up_bytes": gu_bytes,
                  "gate_up_gbs": rate(gu_bytes, gl, gms)})
    if dl:
        r.update({"down_us": dms / dl * 1e3, "down_gbs": rate(dn_bytes, dl, dms)})
    # the dominant kernel: the gate/up launch
    if gl:
        r.update({"dom_kernel": f"k_moe_gate_up<{sfx},{M}>", "dom_us": gms / gl * 1e3,
                  "dom_bytes": gu_bytes, "dom_gbs": rate(gu_bytes, gl, gms)})
    return r


# ------------------------------------------------------- MLA attention --
MFMA_BF16_PEAK_TFLOPS = 2500.0


def mla_bench(U, ctx, torch, steps, warmup, Ts=(1024, 4096, 32768), Rs=(1, 2, 4)):
    """Config 3: absorbed-MLA decode attention at DeepSeek-V3 shape (128
    heads, latent 512 + rope 64, scale 1/sqrt(192)) over an N(0,1) f32 cache,
    R query rows with row s seeing T - R + 1 + s positions.  The cache is
    held on the device in the kernel's split bf16 form (converted once,
    outside the timed region, like a decode session's cache, which is
    appended in that form).  Algorithmic FLOPs 2*128*(576+512) per (row,
    position); bytes = the cache rows read (T*576*4, hi + lo bf16 = the f32
    bytes).  Kernel times are HIP events around each launch on the stream
    the kernels run on."""
    H, L, P = 128, 512, 64
    scale = float(1.0 / np.sqrt(192.0))
    g = torch.Generator(device="cuda:0")
    g.manual_seed(3)
    Tmax = max(Ts)
    lat = torch.randn(Tmax, L, device="cuda:0", generator=g)
    kr = torch.randn(Tmax, P, device="cuda:0", generator=g)
    kc = U.mla_cache_split(ctx, lat, kr)
    del lat, kr
    res = {}
    for R in Rs:
        qabs = torch.randn(R, H, L, device="cuda:0", generator=g)
        qr = torch.randn(R, H, P, device="cuda:0", generator=g)
        out = torch.empty(R, H, L, device="cuda:0")
        for T in Ts:
            pb = T - R
            for _ in range(warmup):
                U.mla_attend_split(ctx, qabs, qr, kc, pb, scale, out=out)
            ctx.synchronize()
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(steps):
                U.mla_attend_split(ctx, qabs, qr, kc, pb, scale, out=out)
            t1.record()
            ctx.synchronize()
            us = t0.elapsed_time(t1) / steps * 1e3
            ctx.enable_timing(True)
            for _ in range(steps):
                U.mla_attend_split(ctx, qabs, qr, kc, pb, scale, out=out)
            ctx.synchronize()
            n1, ms1 = ctx.kernel_time("mla_mfma")
            n2, ms2 = ctx.kernel_time("mla_combine")
            ctx.enable_timing(False)
            flops = 2 * H * (L + P + L) * (R * T - R * (R - 1) // 2)
            nbytes = T * (L + P) * 4
            k_us = ms1 / max(n1, 1) * 1e3
            res[f"R{R}_T{T}"] = {
                "us_per_call": round(us, 2),
                "mfma_kernel_us": round(k_us, 2),
                "combine_us": round(ms2 / max(n2, 1) * 1e3, 2),
                "gflop": round(flops / 1e9, 3),
                "tflops_call": round(flops / (us * 1e-6) / 1e12, 1),
                "mfma_util_call": round(flops / (us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
                "mfma_util_kernel": round(flops / (k_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
                if n1 else None,
                "cache_gbs_call": round(nbytes / (us * 1e-6) / 1e9, 1),
                "hbm_frac_call": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            }
            log(f"config 3 MLA R={R} T={T}: {json.dumps(res[f'R{R}_T{T}'])}")
    del kc
    return res


# --------------------------------------------------------- CPU baseline --
def host_cpu() -> dict:
    """The host the CPU legs run on: model name, ISA flags, cores."""
    info = {"model": None, "flags": [], "nproc": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0))}
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and info["model"] is None:
                info["model"] = line.split(":", 1)[1].strip()
            if line.startswith("flags"):
                fl = set(line.split(":", 1)[1].split())
                info["flags"] = [f for f in ("avx2", "fma", "avx512f", "avx512bw", "avx512_vnni")
                                 if f in fl]
                break
    except OSError:
        pass
    return info


def _timed(fn, min_s: float, min_reps: int = 3):
    fn()
    reps, t0 = 0, time.perf_counter()
    while reps < min_reps or time.perf_counter() - t0 < min_s:
        fn()
        reps += 1
    return (time.perf_counter() - t0) / reps, reps


def cpu_baseline_c2(cfg, seconds):
    """The reference CPU expert block (AVX-512/AVX2 restatement of
    avx512::matmul_i4 with the rayon split, oracle/cpu_baseline.c) on the
    host's cores, M=1, over a 128-expert int4 host pool (2.8 GB, beyond any
    host cache), the same algorithmic bytes per step as the GPU leg."""
    from oracle import oracle as O
    from undertow_amd.configs import expert_bytes
    L = O.cpu_baseline_lib()
    H, I, k = cfg["hidden"], cfg["inter"], cfg["top_k"]
    n = 128
    rng = np.random.default_rng(5)
    gq = rng.integers(0, 256, (n, I, H // 2), dtype=np.uint8)
    uq = rng.integers(0, 256, (n, I, H // 2), dtype=np.uint8)
    dq = rng.integers(0, 256, (n, H, I // 2), dtype=np.uint8)
    gs = (np.abs(rng.normal(0, 0.02, (n, I))) / 7).astype(np.float32)
    us = (np.abs(rng.normal(0, 0.02, (n, I))) / 7).astype(np.float32)
    ds = (np.abs(rng.normal(0, 0.02, (n, H))) / 7).astype(np.float32)
    x = rng.standard_normal((1, H)).astype(np.float32)
    out = np.zeros((1, H), np.float32)
    threads = int(L.ucb_max_threads())
    vp = lambda a: a.ctypes.data

    def step():
        ids = rng.permutation(n)[:k].astype(np.int64)
        w = rng.random(k).astype(np.float32)
        L.ucb_moe_experts(2, H, I, vp(gq), vp(gs), vp(uq), vp(us), vp(dq), vp(ds), 1, k, ids, w,
                          x.reshape(-1), out.reshape(-1), threads)

    dt, steps = _timed(step, seconds, 5)
    isa = {2: "avx512", 1: "avx2", 0: "scalar"}.get(int(L.ucb_isa()), "?")
    return {"value": k * expert_bytes(H, I, 4) / dt / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port", "isa": isa, "ms_per_step": dt * 1e3,
            "sample": f"{steps} steps of the config-2 expert block at M=1 (top-8 over a 128-expert "
                      f"int4 host pool of 2.8 GB, {isa}, {threads} threads), {dt * 1e3:.2f} ms/step"}


def cpu_baseline_c3(seconds_each, Ts=(1024, 4096, 32768), Rs=(1, 2, 4)):
    """Config 3 on the host: the absorbed MLA loops (attention.rs:202-236),
    one task per (row, head) over the host's cores, 128 heads, latent 512 +
    rope 64, at every (R, T)."""
    from oracle import oracle as O
    L = O.cpu_baseline_lib()
    H, Ld, P = 128, 512, 64
    rng = np.random.default_rng(3)
    Tmax = max(Ts)
    lat = rng.standard_normal((Tmax, Ld)).astype(np.float32)
    kr = rng.standard_normal((Tmax, P)).astype(np.float32)
    threads = int(L.ucb_max_threads())
    res = {}
    for R in Rs:
        qabs = rng.standard_normal((R, H, Ld)).astype(np.float32)
        qr = rng.standard_normal((R, H, P)).astype(np.float32)
        out = np.zeros((R, H, Ld), np.float32)
        for T in Ts:
            def call():
                L.ucb_mla_attend(qabs.reshape(-1), qr.reshape(-1), lat.reshape(-1), kr.reshape(-1),
                                 R, H, Ld, P, T - R, 0.0721688, out.reshape(-1), threads)
            dt, reps = _timed(call, seconds_each, 2)
            flops = 2 * H * (Ld + P + Ld) * (R * T - R * (R - 1) // 2)
            res[f"R{R}_T{T}"] = {"us_per_call": round(dt * 1e6, 1), "reps": reps,
                                 "gflops": round(flops / dt / 1e9, 2)}
    return {"unit": "us per call", "cores": threads, "kind": "port", "configs": res}


def cpu_baseline_model(name, cfg, prompt_len, new_tokens, depths, experts=None):
    """Configs 1 and 4 end to end on the host: the oracle's model code over
    the restated dispatched kernels (libcpu_model.so: QTensor::matmul on
    AVX-512/AVX2 with the rayon split, attention tasks per (row, head)),
    greedy and MTP decode tok/s at batch 1, prefill excluded."""
    from oracle import oracle as O
    CM = O.cpu_model_lib()
    over = dict(cfg, init_std=0.02)
    if experts:
        over.update(n_routed_experts=experts)
    sp = O.default_spec(**over)
    t0 = time.perf_counter()
    if name == "c1":
        ck = O.Checkpoint(sp, L=CM)  # the reference's own generator, then converted
        ck.convert(O.INT4, O.INT8)
    else:
        ck = O.Checkpoint.synthesize(sp, 4242, 0.02, O.INT4, O.INT8, L=CM)
    t_make = time.perf_counter() - t0
    m = O.Model(ck)
    rng = np.random.default_rng(42)
    prompt = rng.integers(0, cfg["vocab_size"], prompt_len).tolist()
    t0 = time.perf_counter()
    m.session().prefill(prompt)
    t_prefill = time.perf_counter() - t0
    res = {"prompt": prompt_len, "new_tokens": new_tokens, "make_s": round(t_make, 2),
           "prefill_s": round(t_prefill, 3), "cores": int(O.cpu_baseline_lib().ucb_max_threads()),
           "kind": "port",
           "timing": "decode from the first emitted token to the last (on_token time stamps; "
                     "MTP from the second, after the first round's feed of the prompt)"}

    # Decode rates from time stamps of the emitted tokens: the loops prefill
    # the prompt first, and at config 4 that prefill is ~40x the decode, so
    # subtracting a separately timed prefill would leave mostly its noise.
    # The speculative loop's first round also feeds every prompt position
    # through the MTP layer (prefill work, excluded from the GPU legs' MTP
    # rates too), so its rate starts at the second emitted token.
    def stamped(run, first=0):
        st = []

        def on_token(_t):
            st.append(time.perf_counter())
            return True
        out = run(on_token)
        n = len(st) - first
        return out, (n - 1) / (st[-1] - st[first]) if n > 1 else float("nan")

    toks, tps = stamped(lambda cb: m.generate(prompt, new_tokens, on_token=cb))
    res["greedy_tok_s"] = round(tps, 3)
    for d in depths:
        (mt, drafted, accepted), tps = stamped(
            lambda cb: m.speculative_loop(prompt, new_tokens, depth=d, on_token=cb), first=1)
        res[f"mtp{d}"] = {"tok_s": round(tps, 3), "drafted": drafted,
                          "accepted": accepted, "lossless": mt == toks}
    if experts:
        res["note"] = (f"{experts}-expert pool per layer: the per-token weight bytes are the "
                       f"config's (top-{cfg['num_experts_per_tok']} per layer), the pool is "
                       f"bounded to keep host synthesis short")
    return res


def cpu_baseline(cfg2, seconds=10.0):
    host = host_cpu()
    log(f"CPU baseline host: {host}")
    head = cpu_baseline_c2(cfg2, seconds)
    log(f"CPU config 2: {head['value']:.1f} GB/s")
    head["host"] = host
    legs = {}
    legs["c3"] = cpu_baseline_c3(1.0)
    log(f"CPU config 3: {json.dumps(legs['c3'])}")
    from undertow_amd.configs import C1, C4
    legs["c1"] = cpu_baseline_model("c1", C1, 16, 64, (1,))
    log(f"CPU config 1: {json.dumps(legs['c1'])}")
    # the GPU leg's prompt length (so attention reads the same context); 32
    # tokens keep the leg near ten seconds of host time
    legs["c4"] = cpu_baseline_model("c4", C4, 512, 32, (1,), experts=32)
    log(f"CPU config 4: {json.dumps(legs['c4'])}")
    head["legs"] = legs
    return head


# ------------------------------------------------------------------ MTP --
def model_step_bytes(cfg, rows, unique, ctx_len, expert_bits=4, dense_bits=8, mtp=False):
    """Algorithmic HBM bytes of one forward step of `rows` token rows over the
    main model (and, with mtp, of one MTP-head row): every weight the step
    reads once (int8 dense matrices with f32 row scales, int4 routed
    experts, f32 router gates and norms), `unique` routed experts per MoE
    layer, the compressed KV cache of every layer read once (split bf16 hi/lo
    rows, 2,304 B per position at latent 512 + rope 64), and the activations
    ignored (a few hundred KB)."""
    H, V, L = cfg["hidden_size"], cfg["vocab_size"], cfg["num_hidden_layers"]
    heads, nope, rope, vh = (cfg["num_attention_heads"], cfg["qk_nope_head_dim"],
                             cfg["qk_rope_head_dim"], cfg["v_head_dim"])
    ql, kl, I, Id = cfg["q_lora_rank"], cfg["kv_lora_rank"], cfg["moe_intermediate_size"], \
        cfg["intermediate_size"]
    E = cfg["n_routed_experts"]

    def mat(o, i, bits):
        return o * ((i * bits + 7) // 8) + (o * 4 if bits < 32 else 0)

    attn = (mat(ql, H, dense_bits) + mat(kl + rope, H, dense_bits) +
            mat(heads * (nope + rope), ql, dense_bits) + mat(heads * (nope + vh), kl, dense_bits) +
            mat(H, heads * vh, dense_bits) + 4 * (2 * H + ql + kl))
    kv = ctx_len * (kl + rope) * 4
    expert = 2 * mat(I, H, expert_bits) + mat(H, I, expert_bits)
    Is = I * cfg["n_shared_experts"]
    shared = 2 * mat(Is, H, dense_bits) + mat(H, Is, dense_bits) if Is else 0
    moe = unique * expert + shared + mat(E, H, 32) + 4 * E
    dense = 2 * mat(Id, H, dense_bits) + mat(H, Id, dense_bits)
    nd = cfg["first_k_dense_replace"]
    main = L * (attn + kv) + nd * dense + (L - nd) * moe + mat(V, H, dense_bits) + 4 * H
    if not mtp:
        return main
    head = mat(H, 2 * H, dense_bits) + 4 * 2 * H + attn + kv + moe + mat(V, H, dense_bits) + 4 * H
    return head


def model_roofline(m, cfg, prompt, new_tokens, greedy_tok_s, steps=16):
    """HBM roofline of the DeepSeek-V3-width model's steps: a one-row decode
    step (from the greedy rate: the loop queues each step before reading the
    last token back, so it runs at the GPU's pace) and isolated two- and
    four-row verify steps (host-timed, one readback per step).  Algorithmic
    bytes per model_step_bytes at the run's mean context; one row routes to
    exactly top_k experts per MoE layer, R rows to between top_k and
    R * top_k of them, so the verify figures take top_k (a floor on the
    bytes, hence on the achieved rate) and also give the ceiling."""
    k = cfg["num_experts_per_tok"]
    T = len(prompt) + new_tokens // 2
    b1 = model_step_bytes(cfg, 1, k, T)
    us1 = 1e6 / greedy_tok_s
    out = {"peak_gbs": HBM_PEAK_GBS, "unit": "GB/s",
           "decode": {"bytes": b1, "us_per_step": round(us1, 1),
                      "achieved": round(b1 / us1 / 1e3, 1),
                      "frac": round(b1 / us1 / 1e3 / HBM_PEAK_GBS, 4)}}
    s = m.session()
    s.prefill(prompt, want_logits=False)
    nxt = s.last_argmax[-1]
    # verify rows are distinct tokens, as a verify step's drafts are (a
    # repeated token would route every row to the same experts)
    rng = np.random.default_rng(7)
    for rows in (2, 4):
        s.prefill([nxt] + rng.integers(0, cfg["vocab_size"], rows - 1).tolist(),
                  want_logits=False)  # warm-up of this shape
        nxt = s.last_argmax[-1]
        t0 = time.perf_counter()
        for _ in range(steps):
            s.prefill([nxt] + rng.integers(0, cfg["vocab_size"], rows - 1).tolist(),
                      want_logits=False)
            nxt = s.last_argmax[-1]
        us = (time.perf_counter() - t0) / steps * 1e6
        T = s.position
        lo = model_step_bytes(cfg, rows, k, T)
        hi = model_step_bytes(cfg, rows, min(rows * k, cfg["n_routed_experts"]), T)
        out[f"verify{rows}"] = {"bytes_floor": lo, "bytes_ceiling": hi, "us_per_step": round(us, 1),
                                "achieved_floor": round(lo / us / 1e3, 1),
                                "frac_floor": round(lo / us / 1e3 / HBM_PEAK_GBS, 4),
                                "frac_ceiling": round(hi / us / 1e3 / HBM_PEAK_GBS, 4)}
    del s
    out["mtp_head_bytes"] = model_step_bytes(cfg, 1, k, T, mtp=True)
    return out


def mtp_bench(U, ctx, cfg, prompt_len, new_tokens, depths, seed, expert_fmt, dense_fmt):
    m = U.Model(ctx, cfg)
    t0 = time.perf_counter()
    m.synthesize(seed, 0.02, expert_fmt, dense_fmt)
    ctx.synchronize()
    t_syn = time.perf_counter() - t0
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, cfg["vocab_size"], prompt_len).tolist()
    t_prefill, t_prefill_mtp = prefill_times(m, prompt)
    res = {"device_gb": m.device_bytes / 1e9, "synthesize_s": t_syn, "prefill_s": t_prefill,
           "prefill_with_mtp_feed_s": t_prefill_mtp, "prompt": prompt_len,
           "new_tokens": new_tokens}
    t0 = time.perf_counter()
    greedy = m.generate_greedy(prompt, new_tokens)
    dt = time.perf_counter() - t0 - t_prefill
    res["greedy_tok_s"] = len(greedy) / dt
    if cfg["hidden_size"] >= 4096 and cfg["n_routed_experts"] >= 64:
        res["roofline"] = model_roofline(m, cfg, prompt, new_tokens, res["greedy_tok_s"])
    # the same decode with one-row steps replayed from a captured graph
    before = m.graph_stats()
    m.enable_graphs(True)
    t0 = time.perf_counter()
    greedy_g = m.generate_greedy(prompt, new_tokens)
    dt = time.perf_counter() - t0 - t_prefill
    m.enable_graphs(False)
    after = m.graph_stats()
    assert greedy_g == greedy, "graph replay output differs from the eager decode"
    res["greedy_graph"] = {"tok_s": len(greedy_g) / dt,
                           "replays": after["replays"] - before["replays"],
                           "failures": after["failures"] - before["failures"]}
    for d in depths:
        t0 = time.perf_counter()
        toks, drafted, accepted = m.generate_mtp(prompt, new_tokens, depth=d)
        total = time.perf_counter() - t0
        assert toks == greedy, f"MTP depth {d} output differs from greedy"
        res[f"mtp{d}"] = {"tok_s": len(toks) / (total - t_prefill_mtp), "drafted": drafted,
                          "accepted": accepted, "acceptance": accepted / max(drafted, 1),
                          "lossless": True, "tok_s_with_mtp_feed": len(toks) / (total - t_prefill)}
        # the same loop with its verify steps replayed from a captured graph
        before = m.graph_stats()
        m.enable_graphs(True)
        t0 = time.perf_counter()
        toks_g, _, _ = m.generate_mtp(prompt, new_tokens, depth=d)
        dt = time.perf_counter() - t0 - t_prefill_mtp
        m.enable_graphs(False)
        after = m.graph_stats()
        assert toks_g == greedy, f"MTP depth {d} graph replay output differs from greedy"
        res[f"mtp{d}"]["graph"] = {"tok_s": len(toks_g) / dt,
                                   "replays": after["replays"] - before["replays"],
                                   "failures": after["failures"] - before["failures"]}
        # The accept path's rate: caller drafts (speculative_loop's draft_fn,
        # mtp.rs:263-314) equal to the greedy continuation, so every draft is
        # accepted (the perfect-draft case of pipeline.rs:343-393). Random-init
        # weights give the native head about zero acceptance, so this is the
        # figure that shows what an accepted draft is worth on this step.
        tail = greedy + [0] * (d + 1)

        def perfect(tokens, nxt, dep, _n=len(prompt)):
            e = len(tokens) - _n + 1
            return tail[e:e + dep]

        t0 = time.perf_counter()
        toks_p, drafted_p, accepted_p = m.speculative_loop(prompt, new_tokens, depth=d,
                                                           draft_fn=perfect)
        dt = time.perf_counter() - t0 - t_prefill
        assert toks_p == greedy, f"MTP depth {d} with perfect drafts differs from greedy"
        res[f"mtp{d}"]["perfect_drafts"] = {"tok_s": len(toks_p) / dt, "drafted": drafted_p,
                                            "accepted": accepted_p,
                                            "acceptance": accepted_p / max(drafted_p, 1)}
        # the same with the verify steps replayed from captured graphs
        before = m.graph_stats()
        m.enable_graphs(True)
        t0 = time.perf_counter()
        toks_pg, _, accepted_pg = m.speculative_loop(prompt, new_tokens, depth=d, draft_fn=perfect)
        dt = time.perf_counter() - t0 - t_prefill
        m.enable_graphs(False)
        after = m.graph_stats()
        assert toks_pg == greedy and accepted_pg == accepted_p, \
            f"MTP depth {d} with perfect drafts under graph replay differs"
        res[f"mtp{d}"]["perfect_drafts"]["graph"] = {
            "tok_s": len(toks_pg) / dt, "replays": after["replays"] - before["replays"],
            "failures": after["failures"] - before["failures"]}
    del m
    if cfg["hidden_size"] >= 4096 and cfg.get("mtp"):
        res["restating_head"] = restating_head_bench(U, ctx, cfg, prompt, new_tokens, depths, seed,
                                                     expert_fmt, dense_fmt)
    return res


def prefill_times(m, prompt):
    """(main prefill, main prefill + the MTP module's feed of the prompt),
    seconds, each after a warm-up run: the prefill work the decode rates
    exclude.  The speculative loop's first draft feeds every prompt
    position through the MTP layer (draft_logits over the pending
    positions, mtp.rs:74-133): work proportional to the prompt, done once
    per generation, which a server does at prefill."""
    out = []
    for feed in (False, True):
        for rep in range(2):
            t0 = time.perf_counter()
            s = m.session()
            logits = s.prefill(prompt, want_logits=False)
            if feed:
                s.draft_logits(s.last_argmax[-1])
            dt = time.perf_counter() - t0
            del s, logits
        out.append(dt)
    return out[0], out[1]


def restating_head_bench(U, ctx, cfg, prompt, new_tokens, depths, seed, expert_fmt, dense_fmt):
    """The native draft head at non-zero acceptance: the same config
    synthesized with an MTP module that restates its first MoE layer
    (ut_model_synthesize_ex, UT_SYNTH_MTP_RESTATES; the other layers'
    residual writes damped), so the native head's drafts mostly match the
    verified tokens, as a trained head's do.  The same weight bytes per
    step as the plain model; greedy and MTP depth 1/3 rates (prefill
    excluded), acceptance, and the lossless check."""
    m = U.Model(ctx, cfg)
    m.synthesize(seed, 0.02, expert_fmt, dense_fmt, mtp_restates=True)
    t_prefill, t_prefill_mtp = prefill_times(m, prompt)
    t0 = time.perf_counter()
    greedy = m.generate_greedy(prompt, new_tokens)
    out = {"prefill_s": t_prefill, "prefill_with_mtp_feed_s": t_prefill_mtp,
           "greedy_tok_s": len(greedy) / (time.perf_counter() - t0 - t_prefill)}
    for d in depths:
        t0 = time.perf_counter()
        toks, drafted, accepted = m.generate_mtp(prompt, new_tokens, depth=d)
        total = time.perf_counter() - t0
        assert toks == greedy, f"restating head: MTP depth {d} output differs from greedy"
        tps = len(toks) / (total - t_prefill_mtp)
        out[f"mtp{d}"] = {"tok_s": tps, "drafted": drafted, "accepted": accepted,
                          "acceptance": accepted / max(drafted, 1), "lossless": True,
                          "speedup_vs_greedy": tps / out["greedy_tok_s"],
                          "tok_s_with_mtp_feed": len(toks) / (total - t_prefill)}
    del m
    return out


def c5_bench(U, ctx, torch, prompt_len=2048, new_tokens=256, pin_frac=0.25, cache_frac=0.10,
             seed=42, pool_experts=1024):
    """Config 5: DeepSeek-V3 671B-shaped random-init model at full depth.
    Dense and shared weights (about 18.5 GB int8) are synthesized in HBM; the
    333 GB of int4 routed experts sit behind the expert store's HBM tier,
    filled from a pinned host pool of `pool_experts` seeded experts (key
    (layer, e) reads entry (layer * 256 + e) mod pool_experts: every miss
    moves a real 22 MB expert over the host link).  Two stores:

    - `hbm_rest`: the budget is the HBM left over (about 281 GB).  The
      prompt's prefill records a routing profile, its hottest quarter of all
      routed experts is pinned, then greedy and MTP depth-1 decode of
      `new_tokens` tokens, timed from the first emitted token (prefill
      excluded), with pilot-router prefetch;
    - `streaming`: a budget below the prompt's working set, so the decode
      streams its misses over the host link.  Random-init routing is
      concentrated (the 2048-token prompt touches about a third of the
      14,848 experts), so the BASELINE layout taken over all experts (the
      hottest quarter pinned plus a cache) would hold the whole working
      set; here the hottest `pin_frac` of the experts the profile saw are
      pinned, plus a cache of `cache_frac` of all routed experts.  The same
      greedy and MTP-1 runs, with hit rate and host-link rate."""
    from undertow_amd.configs import C5
    E, nL = C5["n_routed_experts"], C5["num_hidden_layers"] + 1 - C5["first_k_dense_replace"]
    slot = 2 * C5["moe_intermediate_size"] * (C5["hidden_size"] // 2) + \
        C5["hidden_size"] * (C5["moe_intermediate_size"] // 2) + \
        (2 * C5["moe_intermediate_size"] + C5["hidden_size"]) * 4
    n_pin = int(pin_frac * E * nL)
    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, C5["vocab_size"], prompt_len).tolist()
    res = {"prompt": prompt_len, "new_tokens": new_tokens, "host_pool_experts": pool_experts,
           "expert_gb_total": round(E * nL * slot / 1e9, 1), "slot_bytes": slot}

    def store_delta(st0, st1, dt, ntok):
        d = {k: st1[k] - st0[k] for k in ("hits", "misses", "bytes_read", "prefetch_issued",
                                          "evictions")}
        return dict(d, hit_rate=round(d["hits"] / max(d["hits"] + d["misses"], 1), 4),
                    host_link_gbs=round(d["bytes_read"] / dt / 1e9, 2),
                    gb_per_token=round(d["bytes_read"] / max(ntok, 1) / 1e9, 3))

    def decode_runs(m, tag):
        out = {}

        def timed(run):
            stamps = []
            st0 = m.store_stats()
            toks = run(lambda t: stamps.append(time.perf_counter()) or True)
            st1 = m.store_stats()
            dt = stamps[-1] - stamps[0]
            return toks, (len(stamps) - 1) / dt, store_delta(st0, st1, dt, len(toks))

        toks, tps, d = timed(lambda cb: m.generate(prompt, new_tokens, on_token=cb))
        out["greedy_tok_s"] = round(tps, 3)
        out["greedy_store"] = d
        log(f"config 5 {tag} greedy: {out['greedy_tok_s']} tok/s, {json.dumps(d)}")
        counts = {}

        def mtp_run(cb):
            t, counts["drafted"], counts["accepted"] = m.speculative_loop(
                prompt, new_tokens, depth=1, on_token=cb)
            return t

        mt, tps, d = timed(mtp_run)
        out["mtp1"] = {"tok_s": round(tps, 3), **counts, "lossless": mt == toks, "store": d}
        log(f"config 5 {tag} MTP-1: {json.dumps(out['mtp1'])}")
        return out

    free, total = torch.cuda.mem_get_info()
    budget = int(free - 26e9)
    m = U.Model(ctx, C5)
    t0 = time.perf_counter()
    m.synthesize_tiered(seed, budget, pool_experts, prefetch=True)
    ctx.synchronize()
    t_make = time.perf_counter() - t0
    t0 = time.perf_counter()
    s = m.session()
    s.prefill(prompt, want_logits=False)
    t_prefill = time.perf_counter() - t0
    del s
    log(f"config 5: made in {t_make:.1f} s (budget {budget / 1e9:.1f} GB), prompt prefill "
        f"{t_prefill:.1f} s, store {json.dumps(m.store_stats())}")
    usage = m.expert_usage()
    prof = U.ExpertProfile.from_usage("deepseek_v3", usage)
    hot = prof.hottest()
    pinned = m.pin_experts(hot[:n_pin], n_pin * slot)
    r = {"hbm_budget_gb": round(budget / 1e9, 1), "make_s": round(t_make, 2),
         "prefill_s": round(t_prefill, 2), "pinned_gb": round(pinned / 1e9, 1),
         "profiled_experts": len(hot)}
    r.update(decode_runs(m, "hbm_rest"))
    r["evictions"] = m.store_stats()["evictions"]
    res["hbm_rest"] = r
    del m
    torch.cuda.empty_cache()

    # the streaming store: the hottest pin_frac of the profiled experts
    # pinned plus a cache of cache_frac of all experts; the prompt is
    # prefilled through it too
    n_pin = int(pin_frac * len(hot))
    n_cache = int(cache_frac * E * nL)
    sbudget = (n_pin + n_cache) * slot
    m = U.Model(ctx, C5)
    m.synthesize_tiered(seed, sbudget, pool_experts, prefetch=True)
    t0 = time.perf_counter()
    pinned = m.pin_experts(hot[:n_pin], n_pin * slot)
    t_pin = time.perf_counter() - t0
    t0 = time.perf_counter()
    s = m.session()
    s.prefill(prompt, want_logits=False)
    t_prefill = time.perf_counter() - t0
    del s
    log(f"config 5 streaming: budget {sbudget / 1e9:.1f} GB, pinned {pinned / 1e9:.1f} GB in "
        f"{t_pin:.1f} s, prefill {t_prefill:.1f} s")
    r = {"hbm_budget_gb": round(sbudget / 1e9, 1), "pinned_experts": n_pin,
         "cache_experts": n_cache, "pinned_gb": round(pinned / 1e9, 1),
         "cache_gb": round(n_cache * slot / 1e9, 1), "pin_s": round(t_pin, 2),
         "prefill_s": round(t_prefill, 2)}
    r.update(decode_runs(m, "streaming"))
    res["streaming"] = r
    del m
    torch.cuda.empty_cache()
    return res


TRAFFIC_PROFILES = {
    "k_moe_gate_up<int4,1>": "k_moe_gate_up_int4_c2_m1.md",
}


def committed_traffic(kernel: str) -> tuple[float | None, str | None]:
    """HBM bytes per launch of `kernel`, from its committed counter summary:
    rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over this script's
    headline leg, each scaled by what the counter reads for a plain copy of
    known size (--copy-probe).  (None, None) when it is absent."""
    name = TRAFFIC_PROFILES.get(kernel)
    if not name:
        return None, None
    try:
        text = (ROOT / "profiles" / name).read_text()
    except OSError:
        return None, None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.]+)\s*$", text, re.M)
    if not m:
        return None, None
    fs = re.search(r"^fetch_scale:\s*([0-9.]+)\s*$", text, re.M)
    ws = re.search(r"^write_scale:\s*([0-9.]+)\s*$", text, re.M)
    scales = (f"FETCH_SIZE x{fs.group(1)} + WRITE_SIZE x{ws.group(1)}" if fs and ws
              else "FETCH_SIZE + WRITE_SIZE")
    return float(m.group(1)), f"profiles/{name} ({scales} per dispatch, copy-scaled)"



def profile_decode(cfg_name: str, prompt_len: int, tokens: int, seed: int = 42,
                   restating: bool = False) -> None:
    """Decode-step driver for kernel traces (run it under rocprofv3): the
    synthetic model on device, a uniform-random prompt, then `tokens`
    one-row decode steps, `tokens // 2` two-row and `tokens // 2` four-row
    verify steps (the MTP verify widths at depth 1 and 3), the phases
    separated by an idle second so a kernel trace splits cleanly at the
    gaps.  Prints the host-timed ms per step of each phase."""
    import torch
    import undertow_amd as U
    from undertow_amd.configs import C1, C4

    from undertow_amd.configs import C5
    cfg = {"c1": C1, "c4": C4, "c5": C5}[cfg_name]
    ctx = U.Context(0)
    m = U.Model(ctx, cfg)
    if cfg_name == "c5":
        # full depth behind a 40 GB expert tier fed from a 1,024-expert
        # pinned host pool: decode steps read routes back and copy misses
        m.synthesize_tiered(seed, 40 << 30, 1024, prefetch=True)
    else:
        m.synthesize(seed, 0.02, U.INT4, U.INT8, mtp_restates=restating)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, cfg["vocab_size"], prompt_len).tolist()
    s = m.session()
    s.prefill(prompt, want_logits=False)
    nxt = s.last_argmax[-1]
    torch.cuda.synchronize()
    time.sleep(1.0)
    t0 = time.perf_counter()
    for _ in range(tokens):
        s.prefill([nxt], want_logits=False)
        nxt = s.last_argmax[-1]
    t1 = time.perf_counter()
    print(f"decode {tokens} tokens: {(t1 - t0) / tokens * 1e3:.3f} ms/token", flush=True)
    torch.cuda.synchronize()
    time.sleep(1.0)
    n = max(tokens // 2, 1)
    for rows in (2, 4):  # the MTP depth-1 and depth-3 verify widths
        torch.cuda.synchronize()
        time.sleep(1.0)
        t0 = time.perf_counter()
        for _ in range(n):
            # distinct tokens per row, as a verify step's drafts are
            s.prefill([nxt] + rng.integers(0, cfg["vocab_size"], rows - 1).tolist(),
                      want_logits=False)
            nxt = s.last_argmax[-1]
        t1 = time.perf_counter()
        print(f"verify ({rows} rows) {n} steps: {(t1 - t0) / n * 1e3:.3f} ms/step", flush=True)
    if restating:
        # the MTP depth-1 loop with a head that accepts its drafts: verify
        # steps of two rows and the MTP head's feed of the verified rows
        del s
        torch.cuda.synchronize()
        time.sleep(1.0)
        t0 = time.perf_counter()
        toks, drafted, accepted = m.generate_mtp(prompt, tokens, depth=1)
        t1 = time.perf_counter()
        print(f"MTP depth 1: {len(toks)} tokens in {(t1 - t0) * 1e3:.1f} ms (prefill included), "
              f"{accepted}/{drafted} drafts accepted", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--mtp", default="c1,c4", help="comma list of c1,c4 or 'none'")
    ap.add_argument("--c5", action="store_true", default=True,
                    help="config 5 (full depth, experts behind the HBM tier; default on)")
    ap.add_argument("--no-c5", dest="c5", action="store_false")
    ap.add_argument("--c5-tokens", type=int, default=256)
    ap.add_argument("--c5-prompt", type=int, default=2048)
    ap.add_argument("--c5-only", action="store_true",
                    help="only the config 5 leg (no JSON line)")
    ap.add_argument("--variants", action="store_true", default=True)
    ap.add_argument("--no-variants", dest="variants", action="store_false")
    ap.add_argument("--mla", action="store_true", default=True,
                    help="config 3 MLA attention leg (default on)")
    ap.add_argument("--no-mla", dest="mla", action="store_false")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain 1 GiB device copy (counter scaling for rocprofv3 --pmc)")
    ap.add_argument("--read-floor", action="store_true",
                    help="only the single-launch read floor at the expert kernels' sizes "
                         "(fresh windows of a 4 GiB buffer; for kernel traces)")
    ap.add_argument("--mla-only", action="store_true",
                    help="only the config 3 MLA leg (for counter passes; no JSON line)")
    ap.add_argument("--profile-decode", choices=["c1", "c4", "c5"], default=None,
                    help="only run the decode-step driver for kernel traces (no JSON line)")
    ap.add_argument("--prompt", type=int, default=512, help="prompt length for --profile-decode")
    ap.add_argument("--restating", action="store_true",
                    help="--profile-decode: a model whose MTP head restates a layer, plus an "
                         "MTP depth-1 phase")
    ap.add_argument("--tokens", type=int, default=32, help="decode steps for --profile-decode")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only (every GPU box here has "
                                   "one); run with --gpus 1"}))
        sys.exit(2)
    if args.profile_decode:
        profile_decode(args.profile_decode, args.prompt, args.tokens, restating=args.restating)
        return
    if args.c5_only:
        import torch
        import undertow_amd as U
        r = c5_bench(U, U.Context(0), torch, prompt_len=args.c5_prompt, new_tokens=args.c5_tokens)
        print(json.dumps(r), flush=True)
        return
    if args.read_floor:
        import torch
        import undertow_amd as U
        ctx = U.Context(0)
        buf = torch.empty(1 << 30, dtype=torch.int32, device="cuda:0").fill_(1)
        # the expert block's launches: down (8 experts), gate/up (8), both
        for name, nb in (("down_8", 58_982_400), ("gate_up_8", 117_600_256),
                         ("block_8", 176_582_656), ("window_1g", 1 << 30 >> 2)):
            nb = nb // 256 * 256
            g = ctx.probe_read_windows(buf, nb, reps=32)
            print(json.dumps({"window": name, "bytes": nb, "gbs": round(g, 1),
                              "us_per_launch": round(nb / g / 1e3, 2)}), flush=True)
        return
    if args.mla_only:
        import torch
        import undertow_amd as U
        mla_bench(U, U.Context(0), torch, args.steps, args.warmup)
        return

    import torch
    import undertow_amd as U
    from undertow_amd.configs import C1, C2, C4
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    ctx = U.Context(0)

    log("building 256 int4 experts at 7168x2048 on device")
    tbl4 = build_experts(U, ctx, torch, C2["n_experts"], C2["hidden"], C2["inter"], U.INT4, 1)
    head = expert_block_bench(U, ctx, torch, tbl4, C2, 1, args.steps, args.warmup, 4, 11)
    log(f"config 2 int4 M=1: {head['gbs']:.1f} GB/s/step, {head['dom_kernel']} "
        f"{head['dom_gbs']:.1f} GB/s")
    variants = {}
    if args.variants:
        r = expert_block_bench(U, ctx, torch, tbl4, C2, 1, args.steps, args.warmup, 4, 11,
                               fused=False)
        variants["int4_M1_route_then_experts"] = r
        log(f"config 2 int4 M=1, ut_route then ut_moe_experts: {r['gbs']:.1f} GB/s")
        for M in (2, 4):
            r = expert_block_bench(U, ctx, torch, tbl4, C2, M, args.steps, args.warmup, 4, 11 + M)
            variants[f"int4_M{M}"] = r
            log(f"config 2 int4 M={M}: {r['gbs']:.1f} GB/s")
        # the bf16-activation variant of config 2
        for M in (1, 4):
            r = expert_block_bench(U, ctx, torch, tbl4, C2, M, args.steps, args.warmup, 4,
                                   11 + M, bf16x=True)
            variants[f"int4_M{M}_bf16x"] = r
            log(f"config 2 int4 M={M}, bf16 activations: {r['gbs']:.1f} GB/s")
    del tbl4
    torch.cuda.empty_cache()
    if args.variants:
        tbl8 = build_experts(U, ctx, torch, C2["n_experts"], C2["hidden"], C2["inter"], U.INT8, 2)
        # the int8 variant at the same shapes (kernels.rs:21-44)
        for M in (1, 2, 4):
            r = expert_block_bench(U, ctx, torch, tbl8, C2, M, args.steps, args.warmup, 8, 20 + M)
            variants[f"int8_M{M}"] = r
            log(f"config 2 int8 M={M}: {r['gbs']:.1f} GB/s")
        del tbl8
        torch.cuda.empty_cache()

    # measured read ceiling (non-temporal 16-byte loads over 4 GiB)
    buf = torch.empty(1 << 30, dtype=torch.int32, device="cuda:0").fill_(1)
    read_ceiling = ctx.probe_read_bandwidth(buf, reps=10)
    del buf
    torch.cuda.empty_cache()
    log(f"HBM read ceiling (plain read kernel): {read_ceiling:.0f} GB/s")

    if args.copy_probe:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device="cuda:0").fill_(1)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {n} bytes")
        del a, b
        torch.cuda.empty_cache()

    mla = {}
    if args.mla:
        log("config 3 MLA decode attention")
        mla = mla_bench(U, ctx, torch, args.steps, args.warmup)
        torch.cuda.empty_cache()

    mtp = {}
    for name in [n for n in args.mtp.split(",") if n and n != "none"]:
        cfg = {"c1": C1, "c4": C4}[name]
        plen, new = (16, 64) if name == "c1" else (512, 256)
        depths = (1,) if name == "c1" else (1, 3)
        log(f"MTP {name}: prompt {plen}, {new} new tokens, depths {depths}")
        mtp[name] = mtp_bench(U, ctx, cfg, plen, new, depths, 42, U.INT4, U.INT8)
        log(f"MTP {name}: {json.dumps(mtp[name])}")
        torch.cuda.empty_cache()

    c5 = {}
    if args.c5:
        log("config 5: full depth, routed experts behind the expert store's HBM tier")
        c5 = c5_bench(U, ctx, torch, prompt_len=args.c5_prompt, new_tokens=args.c5_tokens)
        log(f"config 5: {json.dumps(c5)}")
        torch.cuda.empty_cache()

    cpu = None
    if not args.skip_cpu:
        log("CPU baseline (reference CPU path restated, host cores)")
        cpu = cpu_baseline(C2)

    dom = head["dom_kernel"]
    traffic, traffic_src = committed_traffic(dom)
    kernels = {k: round(head[k], 3) for k in ("gate_up_us", "down_us", "down_gbs")
               if k in head}
    line = {
        "metric": "MTP accepted tok/s (batch 1) + int4 expert GEMV achieved HBM GB/s vs peak",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 5),
        "host_paced_ms_per_step": round(head["host_paced_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4xf32",
        "data": "synthetic (uniform int4 codes, |N(0,0.02)|/7 row scales, N(0,1) activations and router logits)",
        "config": {"workload": "config 2: int4 routed-expert block, DeepSeek-V3 expert shape "
                               "7168x2048, 256 experts top-8, M=1, fresh routing per step",
                   "hidden": C2["hidden"], "inter": C2["inter"], "experts": C2["n_experts"],
                   "top_k": C2["top_k"], "rows": 1,
                   "unique_experts_per_step": head["unique_experts_mean"],
                   "bytes_per_step": head["bytes_per_step"]},
        "roofline": {"bound": "hbm", "kernel": dom,
                     "achieved": round(head["dom_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["dom_gbs"] / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(head["dom_us"], 3), "bytes_per_launch": head["dom_bytes"],
                     "frac_of_measured_read_ceiling": round(head["dom_gbs"] / read_ceiling, 4),
                     "measured_read_ceiling": round(read_ceiling, 1),
                     "traffic": traffic, "traffic_source": traffic_src},
        "kernels": {**kernels,
                    "all_kernels_us_per_step": round(head["kernels_us_per_step"], 3),
                    "launches_per_step": head["launches_per_step"],
                    # what the bracketing events add to each launch: the
                    # bracketed durations' sum less the queued step time
                    "event_overhead_us_per_launch": round(
                        (head["kernels_us_per_step"] - head["ms_per_step"] * 1e3)
                        / max(head["launches_per_step"], 1), 3)},
        "variants": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                     for k, v in variants.items()},
        "mla": mla,
        "mtp": mtp,
        "c5": c5,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

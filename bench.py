#!/usr/bin/env python3
"""Benchmark: sampled tokens/s of the T3 logits->token sampler at B=256
streams, V=6563 (GPT-2-medium T3 Turbo speech vocabulary), on one MI355X.

A step is one pass of the sampler over one batch: 256 independent streams,
each row 6563 fp32 logits ~N(0,3) with 5 spikes at U[6,12], history length
U[0,1000], temperature U[0.5,1.2], top_k in {50,250,1000}, top_p 0.9,
repetition penalty 1.2, the draw's uniform from the device Philox keyed
(seed, stream, step).  Inputs are synthetic and resident in HBM before timing.
Steps are issued `--steps-per-launch` at a time (one launch samples that many
independent batches; 256 by default, so that the fill at a launch's start and
the drain at its end, about 18% of the time at 64 steps per launch, stay
small); logits rotate over slabs totalling > 2x the 256 MB Infinity Cache so
every step reads its logits from HBM.  `launch_shapes` in the output times
the same kernel at other launch sizes over views of the same slabs.

Prints one JSON line (rank 0) with the headline value, the roofline of the
sampling kernel (algorithmic bytes / measured launch time vs 8 TB/s) and the
CPU baseline (the oracle, the reference's algorithm in C++, on host cores).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

V = 6563
B = 256
HIST_MAX = 1000
HBM_PEAK_GBS = 8000.0
SEED = 0x5EED3


def make_inputs(torch, steps_per_launch, n_slabs, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(SEED)
    slabs = []
    for _ in range(n_slabs):
        x = torch.randn((steps_per_launch * B, V), generator=g, device=dev) * 3.0
        pos = torch.stack([torch.randperm(V, generator=g, device=dev)[:5]
                           for _ in range(8)])  # 8 spike patterns, reused cyclically
        rows = torch.arange(steps_per_launch * B, device=dev)
        pat = pos[rows % 8]
        heights = torch.rand((steps_per_launch * B, 5), generator=g, device=dev) * 6.0 + 6.0
        x.scatter_(1, pat, heights)
        slabs.append(x.contiguous())
    rng = np.random.default_rng(SEED)
    hist = rng.integers(0, V, size=(B, HIST_MAX)).astype(np.int32)
    hist_len = rng.integers(0, HIST_MAX + 1, size=B).astype(np.int32)
    temps = rng.uniform(0.5, 1.2, size=B).astype(np.float32)
    ks = rng.choice(np.array([50, 250, 1000]), size=B)
    params = [dict(top_k=int(ks[r]), top_p=0.9, temp=float(temps[r]), repeat_penalty=1.2,
                   min_p=0.0, cfg_weight=0.0) for r in range(B)]
    return slabs, hist, hist_len, params


def algorithmic_bytes_per_step(hist_len):
    # per row: V fp32 logits + its history ids + 24 B params + 4 B token
    return int(B * (4 * V + 24 + 4) + 4 * int(hist_len.sum()))


def read_traffic(steps_per_launch):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    path = os.path.join(ROOT, "profiles", "sample_rows_b256_v6563_pmc.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("hbm_bytes_per_launch_s%d:" % steps_per_launch):
            return float(line.split(":", 1)[1].split()[0])
    return None


def cpu_baseline(hist, hist_len, params, logits_host, u, gpu_tokens, seconds_1t, seconds_mt):
    import oracle_lib as O
    plist = [O.OParams(p["top_k"], p["top_p"], p["temp"], p["repeat_penalty"], p["min_p"],
                       p["cfg_weight"]) for p in params]
    n_steps = logits_host.shape[0] // B
    out = {}
    # one thread: the reference sampler is single-threaded
    rows = 0
    spent = 0.0
    mism = 0
    s = 0
    while spent < seconds_1t and s < n_steps:
        lg = logits_host[s * B:(s + 1) * B]
        toks, _, secs = O.sample_batch(lg, plist, u[s * B:(s + 1) * B], hist, hist_len,
                                       n_threads=1)
        mism += int(np.sum(toks != gpu_tokens[s * B:(s + 1) * B]))
        rows += B
        spent += secs
        s += 1
    out["1t"] = (rows / spent, rows)
    cores = min(os.cpu_count() or 1, 16)
    rows = 0
    spent = 0.0
    s = 0
    while spent < seconds_mt and s < n_steps:
        k = min(4, n_steps - s)
        lg = logits_host[s * B:(s + k) * B]
        toks, _, secs = O.sample_batch(lg, plist * k, u[s * B:(s + k) * B],
                                       np.tile(hist, (k, 1)), np.tile(hist_len, k),
                                       n_threads=cores)
        mism += int(np.sum(toks != gpu_tokens[s * B:(s + k) * B]))
        rows += k * B
        spent += secs
        s += k
    out["mt"] = (rows / spent, rows, cores)
    out["mismatches"] = mism
    return out


MFMA_F32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
HEAD_EMBD, HEAD_B = 1024, 64


def fused_head_bench(torch, mod, sampler, stream, steps, dev):
    """Q4_0 head + sampler, B=64 CFG pairs (128 projected rows): synthetic
    blocks (random nibbles, fp16 scales of a 0.05-scale weight row) and
    hidden rows, resident in HBM; HIP events on the launch stream."""
    rng = np.random.default_rng(0x4EAD)
    nb = HEAD_EMBD // 32
    blocks = rng.integers(0, 256, size=(V, nb, 18), dtype=np.uint8)
    d = (rng.uniform(0.004, 0.01, size=(V, nb))).astype(np.float16)
    blocks[:, :, :2] = d.view(np.uint8).reshape(V, nb, 2)
    d_w = torch.from_numpy(blocks.reshape(-1)).to(dev)
    d_b = torch.from_numpy((rng.standard_normal(V) * 0.1).astype(np.float32)).to(dev)
    hc = torch.from_numpy(rng.standard_normal((HEAD_B, HEAD_EMBD)).astype(np.float32)).to(dev)
    hu = torch.from_numpy(rng.standard_normal((HEAD_B, HEAD_EMBD)).astype(np.float32)).to(dev)
    lc = torch.empty((HEAD_B, V), dtype=torch.float32, device=dev)
    lu = torch.empty_like(lc)
    head = mod.Sampler.head(d_w, mod.CBX_WTYPE_Q4_0, HEAD_EMBD, hc, lc, bias=d_b,
                            hidden_uncond=hu, logits_uncond=lu)
    w = pkg_workloads()
    plist = [dict(top_k=1000, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.05,
                  cfg_weight=0.5)] * HEAD_B
    d_par = torch.from_numpy(w.pack_params(plist)).to(dev)
    hist = torch.from_numpy(rng.integers(0, V, size=(HEAD_B, 1000)).astype(np.int32)).to(dev)
    hlen = torch.from_numpy(rng.integers(0, 1001, size=HEAD_B).astype(np.int32)).to(dev)
    tok = torch.empty(HEAD_B, dtype=torch.int32, device=dev)

    def fused_step(i):
        sampler.head_sample_batch(head, lc, d_par, tok, history=hist, history_len=hlen,
                                  draw_mode=mod.CBX_DRAW_PHILOX, seed=7, step0=i,
                                  max_survivors=1000)

    def head_only(i):
        sampler.head_logits(head, HEAD_B, V, V)

    res = {}
    for name, fn in (("head", head_only), ("fused", fused_step)):
        for i in range(20):
            fn(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(steps):
            fn(i)
        b.record(stream)
        torch.cuda.synchronize()
        res[name] = a.elapsed_time(b) / steps
    flops = 2.0 * 2 * HEAD_B * V * HEAD_EMBD  # cond and uncond rows
    tf = flops / (res["head"] / 1e3) / 1e12
    return {"workload": "fused Q4_0 speech_head (V=6563 x 1024) + sampler, B=64 CFG pairs "
                        "(128 projected rows), k 1000, p 0.95, T 0.8, pen 1.2, min_p 0.05",
            "steps": steps, "ms_per_step": round(res["fused"], 5),
            "tokens_per_s": round(HEAD_B / (res["fused"] / 1e3), 1),
            "head_ms": round(res["head"], 5),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                         "peak": MFMA_F32_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / MFMA_F32_PEAK_TFLOPS, 4),
                         "kernel": "head_mfma<Q4_0>", "flops_per_launch": flops}}


def pkg_workloads():
    import pkg
    return pkg.workloads()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=16384)
    ap.add_argument("--warmup", type=int, default=1024)
    ap.add_argument("--steps-per-launch", type=int, default=256)
    ap.add_argument("--slabs", type=int, default=2)
    ap.add_argument("--single-launch-steps", type=int, default=200,
                    help="also time this many steps issued one launch per step (0: skip)")
    ap.add_argument("--cpu-seconds", type=float, default=6.0)
    ap.add_argument("--head-steps", type=int, default=200,
                    help="timed steps of the fused speech_head variant (0: skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--shape-steps", type=str, default="16,64",
                    help="also time launches of these many steps (comma list, each dividing "
                         "--steps-per-launch; empty: skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after timing, run a plain device copy of this many MiB (3 times) so "
                         "a counter run can scale FETCH_SIZE / WRITE_SIZE by known bytes")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU; --gpus %d is not supported "
              "(rows are independent and would shard with no exchange)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    import torch
    import pkg

    mod = pkg.load()
    w = pkg.workloads()
    dev = "cuda:0"
    S = args.steps_per_launch
    if args.steps % S or args.warmup % S:
        sys.exit("--steps and --warmup must be multiples of --steps-per-launch")
    slabs, hist, hist_len, params = make_inputs(torch, S, args.slabs, dev)
    d_hist = torch.from_numpy(hist).to(dev)
    d_hlen = torch.from_numpy(hist_len).to(dev)
    d_par = torch.from_numpy(w.pack_params(params)).to(dev)
    sampler = mod.Sampler(device=0, max_vocab=V, max_history=HIST_MAX)
    tokens = torch.empty(S * B, dtype=torch.int32, device=dev)
    philox_seed = 0xC0FFEE

    def launch(slab_idx, step0):
        sampler.sample_batch(slabs[slab_idx], d_par, tokens, n_steps=S, history=d_hist,
                             history_len=d_hlen, draw_mode=mod.CBX_DRAW_PHILOX, seed=philox_seed,
                             step0=step0, max_survivors=1000)

    n_launch_w = args.warmup // S
    n_launch = args.steps // S
    for i in range(n_launch_w):
        launch(i % args.slabs, i * S)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n_launch)]
    t_all0 = torch.cuda.Event(enable_timing=True)
    t_all1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_all0.record(stream)
    for i in range(n_launch):
        ev[i][0].record(stream)
        launch(i % args.slabs, (n_launch_w + i) * S)
        ev[i][1].record(stream)
    t_all1.record(stream)
    torch.cuda.synchronize()
    total_ms = t_all0.elapsed_time(t_all1)
    launch_ms = [a.elapsed_time(b) for a, b in ev]
    avg_launch_ms = float(np.mean(launch_ms))

    steps = n_launch * S
    tok_per_s = steps * B / (total_ms / 1e3)
    bytes_step = algorithmic_bytes_per_step(hist_len)
    bytes_launch = bytes_step * S
    achieved = bytes_launch / (avg_launch_ms / 1e3) / 1e9

    # the same kernel at smaller launch sizes, over views of the same slabs
    shapes = {}
    tokens2 = torch.empty_like(tokens)  # `tokens` keeps the last timed launch for the parity check
    for s2 in [int(x) for x in args.shape_steps.split(",") if x.strip()]:
        if s2 <= 0 or S % s2:
            continue
        per = S // s2
        n2 = max(args.steps // s2, 2 * per)

        def launch2(i):
            sl = slabs[(i // per) % args.slabs][(i % per) * s2 * B:((i % per) + 1) * s2 * B]
            sampler.sample_batch(sl, d_par, tokens2, n_steps=s2, history=d_hist,
                                 history_len=d_hlen, draw_mode=mod.CBX_DRAW_PHILOX,
                                 seed=philox_seed, step0=i * s2, max_survivors=1000)
        for i in range(per):
            launch2(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(n2):
            launch2(i)
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b)
        tps = n2 * s2 * B / (ms / 1e3)
        ach = bytes_step * s2 * n2 / (ms / 1e3) / 1e9
        shapes["s%d" % s2] = {"steps_per_launch": s2, "tokens_per_s": round(tps, 1),
                              "hbm_frac": round(ach / HBM_PEAK_GBS, 5),
                              "ms_per_launch": round(ms / n2, 5)}

    # one launch per step: the decode-loop shape (launch latency included)
    single = None
    if args.single_launch_steps > 0:
        one = slabs[0][:B]
        tok1 = torch.empty(B, dtype=torch.int32, device=dev)
        for i in range(10):
            sampler.sample_batch(one, d_par, tok1, history=d_hist, history_len=d_hlen,
                                 draw_mode=mod.CBX_DRAW_PHILOX, seed=philox_seed, step0=i,
                                 max_survivors=1000)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(args.single_launch_steps):
            sampler.sample_batch(slabs[i % args.slabs][(i % S) * B:(i % S + 1) * B], d_par, tok1,
                                 history=d_hist, history_len=d_hlen,
                                 draw_mode=mod.CBX_DRAW_PHILOX, seed=philox_seed, step0=i,
                                 max_survivors=1000)
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / args.single_launch_steps
        single = {"ms_per_step": round(ms, 5), "tokens_per_s": round(B / (ms / 1e3), 1)}

    # the fused speech_head variant on the B=64 CFG shape: 128 hidden rows
    # (64 cond + 64 uncond) through Q4_0 weights of the Turbo head
    # (V=6563 x 1024), then the sampler over the 64 CFG pairs
    fused = None
    if args.head_steps > 0:
        fused = fused_head_bench(torch, mod, sampler, stream, args.head_steps, dev)

    if args.copy_calibration > 0:
        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    parity = None
    if not args.no_cpu:
        import oracle_lib as O
        # the last timed launch used slab (n_launch-1) % slabs and these steps:
        last_slab = (n_launch - 1) % args.slabs
        step0 = (n_launch_w + n_launch - 1) * S
        gpu_tokens = tokens.cpu().numpy()
        logits_host = slabs[last_slab].cpu().numpy()
        u = np.array([O.philox_uniform(philox_seed, r % B, step0 + r // B)
                      for r in range(S * B)])
        res = cpu_baseline(hist, hist_len, params, logits_host, u, gpu_tokens,
                           args.cpu_seconds, args.cpu_seconds)
        import platform
        model = ""
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
        cpu = {"value": round(res["mt"][0], 1), "unit": "sampled tokens/s",
               "cores": res["mt"][2], "kind": "port",
               "sample": "%d rows (B=256 streams x %d steps of the timed workload) on %d threads; "
                         "single-thread: %.1f tokens/s over %d rows; %s, %s" % (
                             res["mt"][1], res["mt"][1] // B, res["mt"][2], res["1t"][0],
                             res["1t"][1], model, platform.machine()),
               "single_thread_value": round(res["1t"][0], 1)}
        parity = {"rows_checked": res["1t"][1] + res["mt"][1], "token_mismatches": res["mismatches"]}

    out = {
        "metric": "sampled tokens/sec at B=256, V=6563; achieved HBM GB/s vs 8 TB/s peak",
        "value": round(tok_per_s, 1),
        "unit": "sampled tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": n_launch_w * S,
        "ms_per_step": round(total_ms / steps, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch/numpy), resident in HBM",
        "config": {"workload": "batched T3 sampler: B=256 streams, V=6563 fp32 logits, "
                               "top_k {50,250,1000}, top_p 0.9, T U[0.5,1.2], penalty 1.2, "
                               "history U[0,1000], Philox draws",
                   "global_batch": B, "n_vocab": V, "steps_per_launch": S,
                   "logit_slabs_bytes": int(sum(x.numel() * 4 for x in slabs))},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 5),
                     "traffic": read_traffic(S),
                     "kernel": "sample_rows_wave<26,25>",
                     "algorithmic_bytes_per_launch": bytes_launch,
                     "avg_launch_ms": round(avg_launch_ms, 5)},
        "cpu_baseline": cpu,
        "launch_shapes": shapes,
        "single_launch_per_step": single,
        "parity_vs_oracle": parity,
        "fused_head": fused,
    }
    print(json.dumps(out), flush=True)
    sampler.close()


if __name__ == "__main__":
    main()

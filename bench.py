#!/usr/bin/env python3
"""Benchmark: sampled tokens/s of the T3 logits->token sampler at B=256
streams, V=6563 (GPT-2-medium T3 Turbo speech vocabulary), on one MI355X.

A step is one pass of the sampler over one batch: 256 independent streams,
each row 6563 fp32 logits ~N(0,3) with 5 spikes at U[6,12] in random places
of every row, history length U[0,1000], temperature U[0.5,1.2], top_k in
{50,250,1000}, top_p 0.9, repetition penalty 1.2, the draw's uniform from the
device Philox keyed (seed, stream, step).  Inputs are synthetic and resident
in HBM before timing.  Steps are issued `--steps-per-launch` at a time (one
launch samples that many independent batches; 1024 by default, so that the
fill at a launch's start and the drain at its end stay small: 256 read 7%
lower); `--steps` and
`--warmup` are minimums, rounded up to whole launches (at least 64 timed and
32 untimed), and the line reports the steps actually timed.  Logits rotate over slabs totalling > 2x the 256 MB
Infinity Cache so every step reads its logits from HBM.

Prints one JSON line with the headline value, the roofline of the sampling
kernel (algorithmic bytes / measured launch time vs 8 TB/s), the CPU baseline
(the oracle, the reference's algorithm in C++, on host cores) and the other
measured shapes:
  launch_shapes           the same kernel at 16, 64 and 256 steps per launch
  single_launch_per_step  B=256, one launch per step (the decode-loop shape)
  decode_loop             B=256, cbx_decode_step per step with the streams'
                          state on the device, and with a per-token host sync
  configs                 single stream (B=1, V=6563, 500 steps), CFG pair
                          (B=1, V=8194, history growing to 1000), masked
                          stress (B=1024, V=32768, 20% allowed ids)
  fused_head              Q4_0 speech_head + sampler, B=64 CFG pairs
  t3_decode               the T3 transformer's decode step (24 layers, Q4_0)
                          for 64 streams and for 1, alone and with the head and
                          the sampler
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
# The host cores this one-GPU job may use: the host's CPUs are shared among
# its GPUs' jobs, 16 each.
CPU_SHARE = 16


# Fewest launches timed (and run before timing): 16 timed after 4 untimed
# (10 ms of work) read 7% below 64 after 32 (the GPU's clocks still
# ramping); 64 after 32 take about 50 ms.
MIN_TIMED_LAUNCHES = 64
MIN_WARMUP_LAUNCHES = 32


def launches_for(steps, warmup, steps_per_launch):
    """Whole launches covering at least `steps` timed and `warmup` untimed
    steps, and at least MIN_TIMED_LAUNCHES / MIN_WARMUP_LAUNCHES of them:
    (timed launches, warmup launches)."""
    if steps_per_launch < 1:
        raise ValueError("--steps-per-launch must be >= 1")
    n = max(MIN_TIMED_LAUNCHES, -(-max(0, steps) // steps_per_launch))
    nw = max(MIN_WARMUP_LAUNCHES, -(-max(0, warmup) // steps_per_launch))
    return n, nw


def host_threads():
    """(threads used by the CPU baseline, CPUs visible to this process)."""
    try:
        visible = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        visible = os.cpu_count() or 1
    return max(1, min(visible, CPU_SHARE)), visible


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def make_inputs(torch, steps_per_launch, n_slabs, dev):
    g = torch.Generator(device=dev)
    g.manual_seed(SEED)
    slabs = []
    rows = steps_per_launch * B
    for _ in range(n_slabs):
        x = torch.randn((rows, V), generator=g, device=dev) * 3.0
        # 5 spikes per row at random ids; a repeated id keeps the higher spike
        # (a plain scatter of duplicate ids keeps either one, differently from
        # one process to the next)
        pos = torch.randint(0, V, (rows, 5), generator=g, device=dev)
        heights = torch.rand((rows, 5), generator=g, device=dev) * 6.0 + 6.0
        x.scatter_reduce_(1, pos, heights, reduce="amax", include_self=False)
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


def oparams(O, p):
    return O.OParams(p["top_k"], p["top_p"], p["temp"], p["repeat_penalty"], p["min_p"],
                     p["cfg_weight"])


def classify_mismatches(O, rows):
    """rows: (logits, history, params, u, gpu_token, ref_token[, uncond]) of
    every row whose tokens differ.  Returns the counts by class: a
    filter-boundary tie (the oracle flags equal scores across the top-p
    cutoff), a draw-boundary tie (u within 1e-6 of a cumulative boundary of
    the oracle's probabilities) or a hard mismatch."""
    import parity
    out = {"hard": 0, "filter_ties": 0, "draw_ties": 0}
    for r in rows:
        lg, h, p, u, _, _ = r[:6]
        un = r[6] if len(r) > 6 else None
        _, info, probs, _ = O.sample_row(lg, h, oparams(O, p), u, uncond=un, want_probs=True)
        if info & O.INFO_TOPP_TIE:
            out["filter_ties"] += 1
        elif parity._near_cdf_boundary(probs, u):
            out["draw_ties"] += 1
        else:
            out["hard"] += 1
    return out


def cpu_baseline(O, hist, hist_len, params, logits_host, u, gpu_tokens, seconds_1t, seconds_mt,
                 threads):
    plist = [oparams(O, p) for p in params]
    n_steps = logits_host.shape[0] // B
    out = {}
    bad_rows = {}
    checked = set()

    def check(s0, k, toks):
        want = gpu_tokens[s0 * B:(s0 + k) * B]
        checked.update(range(s0, s0 + k))
        for i in np.nonzero(toks != want)[0]:
            r = s0 * B + int(i)
            q = r % B
            bad_rows[r] = (logits_host[r], hist[q][:hist_len[q]], params[q], u[r],
                           int(want[i]), int(toks[i]))

    # one thread: the reference sampler is single-threaded
    rows, spent, s = 0, 0.0, 0
    while spent < seconds_1t and s < n_steps:
        lg = logits_host[s * B:(s + 1) * B]
        toks, _, secs = O.sample_batch(lg, plist, u[s * B:(s + 1) * B], hist, hist_len,
                                       n_threads=1)
        check(s, 1, toks)
        rows += B
        spent += secs
        s += 1
    out["1t"] = (rows / spent, rows)
    # all threads, over the same steps again from the first (and around
    # again while the time lasts)
    rows, spent, s = 0, 0.0, 0
    while spent < seconds_mt:
        s %= n_steps
        k = min(16, n_steps - s)
        lg = logits_host[s * B:(s + k) * B]
        toks, _, secs = O.sample_batch(lg, plist * k, u[s * B:(s + k) * B],
                                       np.tile(hist, (k, 1)), np.tile(hist_len, k),
                                       n_threads=threads)
        check(s, k, toks)
        rows += k * B
        spent += secs
        s += k
    out["mt"] = (rows / spent, rows) if rows else (0.0, 0)
    out["rows_checked"] = len(checked) * B
    out["mismatch"] = len(bad_rows)
    out["classes"] = classify_mismatches(O, list(bad_rows.values()))
    return out


def timed(torch, stream, fn, n, warm=3):
    """Mean ms per call of fn(i) over n calls, by HIP events on `stream`."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(n):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def decode_loop_bench(torch, mod, sampler, dev, slabs, S, d_par, hist, hist_len, steps, seed):
    """B=256 streams of the engine's decode loop, one cbx_decode_step per step
    on logits taken from the slabs (the step graph's output left on the
    device): each stream's history grows on the device and nothing is copied
    to the host between steps.  Beside it, the same loop with the reference's
    per-token host round trip: the step's tokens copied to the host and waited
    for before the next step is issued.  The stop id lies outside the
    vocabulary so every stream is sampled at every step.  Wall clock over the
    timed steps."""
    ld = int(hist_len.max()) + steps + 64
    h0 = np.zeros((B, ld), np.int32)
    h0[:, :hist.shape[1]] = hist
    warm, res, grew = 10, {}, True
    for mode in ("device", "host_sync"):
        dh = torch.from_numpy(h0).to(dev)
        dl = torch.from_numpy(hist_len).to(dev)
        st = torch.zeros(B, dtype=torch.int32, device=dev)
        nxt = torch.zeros(B, dtype=torch.int32, device=dev)
        tok = torch.empty(B, dtype=torch.int32, device=dev)
        host = torch.empty(B, dtype=torch.int32, pin_memory=True)
        dec = mod.Sampler.decode_state(st, dh, dl, next_token=nxt)
        cur = torch.cuda.current_stream()

        def step(i):
            sampler.decode_step(slabs[i % len(slabs)][(i % S) * B:(i % S + 1) * B], d_par, tok,
                                dec, draw_mode=mod.CBX_DRAW_PHILOX, seed=seed, step0=i,
                                stop_token=-1)
            if mode == "host_sync":
                host.copy_(tok, non_blocking=True)
                cur.synchronize()
        for i in range(warm):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            step(warm + i)
        torch.cuda.synchronize()
        res[mode] = (time.perf_counter() - t0) * 1e3 / steps
        grew = grew and bool(np.array_equal(dl.cpu().numpy(), hist_len + warm + steps)) and \
            int(st.abs().sum().item()) == 0
    return {"workload": "decode loop, B=256 streams, V=6563, one cbx_decode_step per step "
                        "(history grows on the device)",
            "steps": steps,
            "ms_per_step_device": round(res["device"], 5),
            "ms_per_step_host_sync": round(res["host_sync"], 5),
            "tokens_per_s_device": round(B / (res["device"] / 1e3), 1),
            "histories_grew_by_steps": grew}


T3_LAYER, T3_EMBD, T3_HEAD = 24, 1024, 16  # GPT-2 medium, the Turbo T3


def q4_0_rows(torch, rows, n_in, dev, g):
    """Random Q4_0 matrix bytes [rows][n_in/32 blocks of 18]: fp16 scales in
    [0.001, 0.004] (weights of about N(0, 0.02)), random nibbles."""
    nb = n_in // 32
    b = torch.randint(0, 256, (rows, nb, 18), generator=g, device=dev, dtype=torch.uint8)
    d = (torch.rand((rows, nb), generator=g, device=dev) * 0.003 + 0.001).half()
    b[:, :, :2] = d.contiguous().view(torch.uint8).view(rows, nb, 2)
    return b.reshape(-1)


def t3_parity(torch, O, sampler, model, layers, wpe, emb, lnf, kc, vc, pos, hid, check, V):
    """One more cbx_t3_step at the timed shape (every stream at the position
    the timed steps left it) against the binary64 oracle for the streams in
    `check`: their caches copied as the device holds them, the matrices
    dequantized from the device's Q4_0 bytes.  Returns the largest error of
    ln_f's rows and whether every row is within 5e-5 + 5e-5 |ref|."""
    from oracle import cbx_t3_oracle as T3
    n = T3_EMBD
    B = pos.numel()
    g = torch.Generator(device=kc.device)
    g.manual_seed(0x7334)
    toks = torch.randint(0, V, (B,), generator=g, device=kc.device, dtype=torch.int32)
    p = pos.cpu().numpy().astype(np.int64)
    assert np.all(p == p[0]) and p[0] + 1 < kc.shape[-2]
    sampler.t3_step(model, pos, kc, vc, hid, tokens=toks)
    torch.cuda.synchronize()
    got = hid.cpu().numpy()[check]
    deq = lambda w, o, i: O.dequantize(w.cpu().numpy().reshape(o, -1), O.WTYPE_Q4_0, i)
    host = lambda t: t.cpu().numpy()
    ref_layers = [dict(ln_1_g=host(L["ln_1_g"]), ln_1_b=host(L["ln_1_b"]),
                       attn_w=deq(L["attn_w"], 3 * n, n), attn_b=host(L["attn_b"]),
                       attn_proj_w=deq(L["attn_proj_w"], n, n),
                       attn_proj_b=host(L["attn_proj_b"]), ln_2_g=host(L["ln_2_g"]),
                       ln_2_b=host(L["ln_2_b"]), fc_w=deq(L["fc_w"], 4 * n, n),
                       fc_b=host(L["fc_b"]), fc_proj_w=deq(L["fc_proj_w"], n, 4 * n),
                       fc_proj_b=host(L["fc_proj_b"])) for L in layers]
    rm = T3.Model(ref_layers, host(wpe), host(emb), host(lnf[0]), host(lnf[1]), 1e-5, T3_HEAD)
    L = int(p[0]) + 1
    # the device caches after the step: position p[0] holds the step's own k
    # and v, which the oracle writes again from its own products
    kr = T3.StreamCaches([host(kc[r, :, :, :L]) for r in check])
    vr = T3.StreamCaches([host(vc[r, :, :, :L]) for r in check])
    want = T3.step(rm, host(toks)[check], p[check].copy(), kr, vr)
    err = np.abs(got.astype(np.float64) - want)
    ok = bool(np.all(err <= 5e-5 + 5e-5 * np.abs(want)))
    return {"streams_checked": [int(r) for r in check], "position": int(p[0]),
            "max_abs_err": float(err.max()), "tol": "5e-5 + 5e-5 |ref| on ln_f rows",
            "ok": ok}


def t3_bench(torch, mod, sampler, dev, B, pos0, n_ctx, steps, O=None):
    """The T3 decode step (cbx_t3_step) of B streams on the Turbo shape with
    random Q4_0 matrices, every stream at position pos0 (caches of n_ctx
    positions), alone and followed by the fused Q4_0 speech_head and the
    sampler (cbx_head_decode_step): the whole device decode step.  Bytes per
    step: the layer matrices once, every stream's K and V read over its
    positions and the new row written.  With the oracle (O), one more step at
    the timed shape is checked against it (t3_parity)."""
    assert pos0 + steps + 1 < n_ctx, "every timed step and the checked one fit the caches"
    g = torch.Generator(device=dev)
    g.manual_seed(0x7333)
    n = T3_EMBD
    vec = lambda k, base=0.0, sd=0.1: (base + torch.randn(k, generator=g, device=dev) * sd)
    layers = [dict(ln_1_g=vec(n, 1.0), ln_1_b=vec(n), attn_w=q4_0_rows(torch, 3 * n, n, dev, g),
                   attn_b=vec(3 * n, 0.0, 0.02), attn_proj_w=q4_0_rows(torch, n, n, dev, g),
                   attn_proj_b=vec(n, 0.0, 0.02), ln_2_g=vec(n, 1.0), ln_2_b=vec(n),
                   fc_w=q4_0_rows(torch, 4 * n, n, dev, g), fc_b=vec(4 * n, 0.0, 0.02),
                   fc_proj_w=q4_0_rows(torch, n, 4 * n, dev, g), fc_proj_b=vec(n, 0.0, 0.02))
              for _ in range(T3_LAYER)]
    wpe = vec(n_ctx * n, 0.0, 0.1).view(n_ctx, n)
    emb = vec(V * n, 0.0, 0.5).view(V, n)
    model = mod.Sampler.t3_model(layers, wpe, emb, vec(n, 1.0), vec(n), wtype=mod.CBX_WTYPE_Q4_0,
                                 n_head=T3_HEAD)
    kc = torch.randn((B, T3_LAYER, T3_HEAD, n_ctx, 64), generator=g, device=dev) * 0.5
    vc = torch.randn((B, T3_LAYER, T3_HEAD, n_ctx, 64), generator=g, device=dev) * 0.5
    hid = torch.empty((B, n), dtype=torch.float32, device=dev)
    pos = torch.full((B,), pos0, dtype=torch.int32, device=dev)
    toks = torch.randint(0, V, (B,), generator=g, device=dev, dtype=torch.int32)
    head_w = q4_0_rows(torch, V, n, dev, g)
    head_b = vec(V, 0.0, 0.1)
    logits = torch.empty((B, V), dtype=torch.float32, device=dev)
    head = mod.Sampler.head(head_w, mod.CBX_WTYPE_Q4_0, n, hid, logits, bias=head_b)
    w = pkg_workloads()
    prm = torch.from_numpy(w.pack_params([dict(top_k=1000, top_p=0.95, temp=0.8,
                                                repeat_penalty=1.2, min_p=0.0,
                                                cfg_weight=0.0)] * B)).to(dev)
    state = torch.zeros(B, dtype=torch.int32, device=dev)
    hist = torch.zeros((B, steps + 16), dtype=torch.int32, device=dev)
    hlen = torch.zeros(B, dtype=torch.int32, device=dev)
    tok_out = torch.empty(B, dtype=torch.int32, device=dev)
    dec = mod.Sampler.decode_state(state, hist, hlen, next_token=toks)
    stream = torch.cuda.current_stream()
    res = {}
    for name in ("t3", "t3_head_sampler"):
        def one(i, name=name):
            if i == 0:
                pos.fill_(pos0)
                hlen.zero_()
            sampler.t3_step(model, pos, kc, vc, hid, tokens=toks, state=state)
            if name != "t3":
                sampler.decode_step(logits, prm, tok_out, dec, head=head, seed=7, step0=i,
                                    stop_token=-1)
        res[name] = timed(torch, stream, one, steps, warm=1)
        # every stream stepped at every timed call (none ran out of cache)
        assert np.all(pos.cpu().numpy() == pos0 + steps)
    parity = None
    if O is not None:
        check = [0, B - 1] if B > 1 else [0]
        parity = t3_parity(torch, O, sampler, model, layers, wpe, emb, (model._keep[4],
                                                                         model._keep[5]),
                           kc, vc, pos, hid, check, V)
    # the prompt pass: every stream's first pos0 positions in one call
    P = min(pos0, n_ctx)
    slots = torch.arange(B, device=dev, dtype=torch.int32).repeat_interleave(P)
    ppos = torch.arange(P, device=dev, dtype=torch.int32).repeat(B)
    prow = torch.randn((B * P, n), generator=g, device=dev) * 0.5
    phid = torch.empty((B * P, n), dtype=torch.float32, device=dev)
    res["prefill"] = timed(torch, stream, lambda i: sampler.t3_prefill(
        model, slots, ppos, kc, vc, phid, inputs=prow), 3, warm=1)
    mat_bytes = T3_LAYER * 12 * n * n * 18 // 32
    # per step and stream: K and V read over positions [0, pos] (pos0 .. pos0
    # + steps - 1 over the timed steps) and written at pos, every layer
    mean_pos = pos0 + (steps - 1) / 2.0
    kv_bytes = B * T3_LAYER * 2 * n * 4 * (mean_pos + 2)
    bytes_step = mat_bytes + kv_bytes
    ms = res["t3"]
    return {"workload": "T3 decode step, GPT-2 medium (24 layers, 1024, 16 heads), Q4_0 "
                        "matrices, %d streams at positions %d-%d, fp32 KV caches" % (
                            B, pos0, pos0 + steps),
            "streams": B, "steps": steps,
            "ms_per_step_t3": round(ms, 5),
            "ms_per_step_with_head_and_sampler": round(res["t3_head_sampler"], 5),
            "tokens_per_s": round(B / (res["t3_head_sampler"] / 1e3), 1),
            "algorithmic_bytes_per_step": int(bytes_step),
            "hbm_frac_t3": round(bytes_step / (ms / 1e3) / 1e9 / HBM_PEAK_GBS, 5),
            "parity_vs_oracle": parity,
            "prefill": {"rows": B * P, "positions_per_stream": P,
                        "ms": round(res["prefill"], 4),
                        "positions_per_s": round(B * P / (res["prefill"] / 1e3), 1)}}


def pkg_workloads():
    import pkg
    return pkg.workloads()


MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix peak
HEAD_EMBD, HEAD_B = 1024, 64


def fused_head_bench(torch, mod, sampler, stream, steps, dev):
    """Q4_0 head + sampler, B=64 CFG pairs (128 projected rows): synthetic
    blocks (random nibbles, fp16 scales of a 0.05-scale weight row) and
    hidden rows, resident in HBM; HIP events on the launch stream.  Also the
    projection of one CFG pair alone (2 rows), the single-stream shape."""
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

    def head_pair(i):
        sampler.head_logits(head, 1, V, V)

    res = {}
    for name, fn in (("head", head_only), ("fused", fused_step), ("pair", head_pair)):
        res[name] = timed(torch, stream, fn, steps, warm=20)
    flops = 2.0 * 2 * HEAD_B * V * HEAD_EMBD  # cond and uncond rows
    # the fraction on the projection's own FLOPs; the fp16 matrix cores take
    # each activation as two parts (hi, lo), so they execute twice as many;
    # the split pre-pass and launch gaps are inside the timed call
    tf = flops / (res["head"] / 1e3) / 1e12
    return {"workload": "fused Q4_0 speech_head (V=6563 x 1024) + sampler, B=64 CFG pairs "
                        "(128 projected rows), k 1000, p 0.95, T 0.8, pen 1.2, min_p 0.05",
            "steps": steps, "ms_per_step": round(res["fused"], 5),
            "tokens_per_s": round(HEAD_B / (res["fused"] / 1e3), 1),
            "head_ms": round(res["head"], 5),
            "head_one_cfg_pair_ms": round(res["pair"], 5),
            "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                         "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                         "kernel": "head_split + head_mfma<Q4_0,2>",
                         "flops_per_launch": flops, "fp16_flops_per_launch": 2 * flops}}


def config_single_stream(torch, mod, sampler, stream, dev, O):
    """B=1, V=6563, 500 steps, fixed history of 256 ids; k 1000, p 0.95,
    T 0.8, pen 1.2, min_p 0.05.  Philox draws keyed (seed, stream 0, step)."""
    w = pkg_workloads()
    d = w.single_stream(steps=500, min_p=0.05)
    n = d["logits"].shape[0]
    lg = torch.from_numpy(d["logits"]).to(dev)
    hist = torch.from_numpy(d["history"][None, :]).to(dev)
    hl = torch.tensor([d["history"].size], dtype=torch.int32, device=dev)
    prm = torch.from_numpy(w.pack_params([d["params"]])).to(dev)
    tok = torch.empty(n, dtype=torch.int32, device=dev)
    seed = 0x51
    u = np.array([O.philox_uniform(seed, 0, t) for t in range(n)]) if O else None

    # top_k 1000 bounds the survivors by 1000 (rows with more, from ties at
    # the k-th score, are sampled again at full capacity by the redo pass)
    def step(i, hint=1000):
        t = i % n
        sampler.sample_batch(lg[t:t + 1], prm, tok[t:t + 1], history=hist, history_len=hl,
                             draw_mode=mod.CBX_DRAW_PHILOX, seed=seed, step0=t,
                             max_survivors=hint)

    ms_nohint = timed(torch, stream, lambda i: step(i, 0), n)
    got_nohint = tok.cpu().numpy()
    ms_batch = timed(torch, stream, step, n)
    got = tok.cpu().numpy()
    assert np.array_equal(got, got_nohint), "survivor hint changed tokens"

    def all_steps(i):
        sampler.sample_batch(lg, prm, tok, n_steps=n, history=hist, history_len=hl,
                             draw_mode=mod.CBX_DRAW_PHILOX, seed=seed, step0=0,
                             max_survivors=1000)

    ms_all = timed(torch, stream, all_steps, 5, warm=1)
    # the row API: host logits in, token out (PCIe copies included)
    host = d["logits"]
    t0 = time.perf_counter()
    for t in range(100):
        sampler.sample_row(host[t], d["history"], d["params"], u[t] if u is not None else 0.5)
    ms_row = (time.perf_counter() - t0) * 1e3 / 100
    out = {"workload": "B=1, V=6563, 500 steps, history 256, k 1000, p 0.95, T 0.8, pen 1.2, "
                       "min_p 0.05",
           "us_per_step_batch_api": round(ms_batch * 1e3, 2),
           "us_per_step_batch_api_no_survivor_hint": round(ms_nohint * 1e3, 2),
           "us_per_step_one_launch_500_steps": round(ms_all * 1e3 / n, 3),
           "us_per_step_row_api_pcie": round(ms_row * 1e3, 2)}
    if O is not None:
        ref, _, secs = O.sample_batch(d["logits"], [oparams(O, d["params"])] * n, u,
                                      np.tile(d["history"], (n, 1)),
                                      np.full(n, d["history"].size, np.int32), n_threads=1)
        bad = [(d["logits"][t], d["history"], d["params"], u[t], int(got[t]), int(ref[t]))
               for t in np.nonzero(got != ref)[0]]
        out["cpu_us_per_step_1t"] = round(secs * 1e6 / n, 2)
        out["parity_vs_oracle"] = dict(rows_checked=n, token_mismatches=len(bad),
                                       **classify_mismatches(O, bad))
    return out


def config_cfg_pair(torch, mod, sampler, stream, dev, O, steps=1000):
    """CFG pair, B=1, V=8194, 1000 steps: cond ~N(0,3), uncond = cond + N(0,1),
    w 0.5, top-k off, p 0.95, T 0.8, pen 1.2, min_p 0.05; the history at step t
    is the t tokens drawn before it (the oracle's sequence, Philox uniforms)."""
    w = pkg_workloads()
    d = w.cfg_pair(steps=steps)
    seed = 0xCF6
    p = d["params"]
    seq = []
    cpu_s = 0.0
    if O is not None:
        op = oparams(O, p)
        for t in range(steps):
            t0 = time.perf_counter()
            tk, _ = O.sample_row(d["cond"][t], seq, op, O.philox_uniform(seed, 0, t),
                                 uncond=d["uncond"][t])
            cpu_s += time.perf_counter() - t0
            seq.append(tk)
    else:
        seq = list(np.random.default_rng(1).integers(0, d["V"], size=steps))
    hist = torch.from_numpy(np.array(seq, np.int32)[None, :]).to(dev)
    hls = torch.arange(steps, dtype=torch.int32, device=dev)
    c = torch.from_numpy(d["cond"]).to(dev)
    un = torch.from_numpy(d["uncond"]).to(dev)
    prm = torch.from_numpy(w.pack_params([p])).to(dev)
    tok = torch.empty(steps, dtype=torch.int32, device=dev)

    def step(i):
        t = i % steps
        sampler.sample_batch(c[t:t + 1], prm, tok[t:t + 1], logits_uncond=un[t:t + 1],
                             history=hist, history_len=hls[t:t + 1],
                             draw_mode=mod.CBX_DRAW_PHILOX, seed=seed, step0=t)

    ms = timed(torch, stream, step, steps)
    got = tok.cpu().numpy()
    out = {"workload": "CFG pair B=1, V=8194, 1000 steps, history growing 0->999, top-k off, "
                       "p 0.95, T 0.8, pen 1.2, min_p 0.05, w 0.5",
           "us_per_step_batch_api": round(ms * 1e3, 2)}
    if O is not None:
        ref = np.array(seq, np.int32)
        bad = [(d["cond"][t], seq[:t], p, O.philox_uniform(seed, 0, t), int(got[t]),
                int(ref[t]), d["uncond"][t]) for t in np.nonzero(got != ref)[0]]
        out["cpu_us_per_step_1t"] = round(cpu_s * 1e6 / steps, 2)
        out["parity_vs_oracle"] = dict(rows_checked=steps, token_mismatches=len(bad),
                                       **classify_mismatches(O, bad))
    return out


def config_masked_stress(torch, mod, sampler, stream, dev, steps=48, n_slabs=4):
    """B=1024, V=32768 logits ~N(0,4), allowed bitmask with 20% of ids set,
    forced stop on 1/16 of the rows, history 512, pen 1.3, k 50, p 0.9,
    min_p 0.02; one launch per step over slabs of 128 MiB rotating through
    512 MiB (twice the Infinity Cache)."""
    Bm, Vm, H = 1024, 32768, 512
    Wm = Vm // 32
    g = torch.Generator(device=dev)
    g.manual_seed(0x5EED5)
    slabs = [(torch.randn((Bm, Vm), generator=g, device=dev) * 4.0).contiguous()
             for _ in range(n_slabs)]
    bits = (torch.rand((Bm, Wm, 32), generator=g, device=dev) < 0.2).to(torch.int64)
    stop = Vm - 1
    bits[:, stop // 32, stop % 32] = 1
    words = (bits << torch.arange(32, device=dev, dtype=torch.int64)).sum(-1)
    allowed = words.to(torch.int64).bitwise_and(0xFFFFFFFF)
    allowed = torch.where(allowed >= 2**31, allowed - 2**32, allowed).to(torch.int32).contiguous()
    force = (torch.rand(Bm, generator=g, device=dev) < 1.0 / 16).to(torch.uint8)
    hist = torch.randint(0, Vm, (Bm, H), generator=g, device=dev, dtype=torch.int32)
    hl = torch.full((Bm,), H, dtype=torch.int32, device=dev)
    w = pkg_workloads()
    prm = torch.from_numpy(w.pack_params([dict(top_k=50, top_p=0.9, temp=0.8,
                                               repeat_penalty=1.3, min_p=0.02,
                                               cfg_weight=0.0)] * Bm)).to(dev)
    tok = torch.empty(Bm, dtype=torch.int32, device=dev)
    info = torch.zeros(Bm, dtype=torch.int32, device=dev)

    def step(i):
        sampler.sample_batch(slabs[i % n_slabs], prm, tok, history=hist, history_len=hl,
                             allowed=allowed, force_stop=force, stop_token=stop, info=info,
                             draw_mode=mod.CBX_DRAW_PHILOX, seed=5, step0=i, max_survivors=50)

    ms = timed(torch, stream, step, steps, warm=n_slabs)
    bytes_step = Bm * (4 * Vm + 4 * H + Wm * 4 + 1 + 24 + 8)
    gbs = bytes_step / (ms / 1e3) / 1e9
    flags = info.cpu().numpy().view(np.uint32)
    return {"workload": "masked stress B=1024, V=32768, 20% allowed, forced stop 1/16, "
                        "history 512, k 50, p 0.9, min_p 0.02, pen 1.3",
            "us_per_step": round(ms * 1e3, 2),
            "tokens_per_s": round(Bm / (ms / 1e3), 1),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 5),
                         "algorithmic_bytes_per_step": bytes_step,
                         "kernel": "sample_rows_wave<128,0,true,true> (the row read in chunks by two waves)"},
            "overflow_rows": int(np.sum((flags & 0x20) != 0))}


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=65536,
                    help="timed steps (at least; rounded up to whole launches)")
    ap.add_argument("--warmup", type=int, default=1024,
                    help="untimed steps first (at least; rounded up to whole launches)")
    ap.add_argument("--steps-per-launch", type=int, default=1024)
    ap.add_argument("--slabs", type=int, default=2)
    ap.add_argument("--latency-rows", type=int, default=None,
                    help="the sampler's small-launch rule: calls of at most this many row-steps "
                         "run the workgroup kernel (library default 512; 0: never)")
    ap.add_argument("--single-launch-steps", type=int, default=200,
                    help="also time this many steps issued one launch per step (0: skip)")
    ap.add_argument("--t3-steps", type=int, default=20,
                    help="timed steps of the T3 decode step, B=64 and B=1 (0: skip)")
    ap.add_argument("--decode-steps", type=int, default=200,
                    help="timed steps of the device decode loop and its host-synced twin "
                         "(0: skip)")
    ap.add_argument("--cpu-seconds", type=float, default=6.0,
                    help="wall seconds of the single-thread CPU baseline")
    ap.add_argument("--cpu-mt-seconds", type=float, default=2.0,
                    help="wall seconds of the all-threads CPU baseline")
    ap.add_argument("--head-steps", type=int, default=200,
                    help="timed steps of the fused speech_head variant (0: skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations (single stream, CFG pair, masked)")
    ap.add_argument("--shape-steps", type=str, default="16,64,256",
                    help="also time launches of these many steps (comma list; entries that do "
                         "not divide --steps-per-launch are skipped; empty: skip)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after timing, run a plain device copy of this many MiB (3 times) so "
                         "a counter run can scale FETCH_SIZE / WRITE_SIZE by known bytes")
    return ap.parse_args(argv)


def main():
    args = parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU; --gpus %d is not supported "
              "(rows are independent and would shard with no exchange)" % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    t_start = time.perf_counter()
    import torch
    import pkg

    mod = pkg.load()
    w = pkg.workloads()
    dev = "cuda:0"
    S = args.steps_per_launch
    n_launch, n_launch_w = launches_for(args.steps, args.warmup, S)
    slabs, hist, hist_len, params = make_inputs(torch, S, args.slabs, dev)
    d_hist = torch.from_numpy(hist).to(dev)
    d_hlen = torch.from_numpy(hist_len).to(dev)
    d_par = torch.from_numpy(w.pack_params(params)).to(dev)
    sampler = mod.Sampler(device=0, max_vocab=32768, max_history=HIST_MAX)
    if args.latency_rows is not None:
        sampler.set_latency_rows(args.latency_rows)
    tokens = torch.empty(S * B, dtype=torch.int32, device=dev)
    philox_seed = 0xC0FFEE

    def launch(slab_idx, step0):
        sampler.sample_batch(slabs[slab_idx], d_par, tokens, n_steps=S, history=d_hist,
                             history_len=d_hlen, draw_mode=mod.CBX_DRAW_PHILOX, seed=philox_seed,
                             step0=step0, max_survivors=1000)

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
        # the slab after the one the previous launch read
        launch((n_launch_w + i) % args.slabs, (n_launch_w + i) * S)
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
        n2 = max(4096 // s2, 2 * per)

        def launch2(i):
            sl = slabs[(i // per) % args.slabs][(i % per) * s2 * B:((i % per) + 1) * s2 * B]
            sampler.sample_batch(sl, d_par, tokens2, n_steps=s2, history=d_hist,
                                 history_len=d_hlen, draw_mode=mod.CBX_DRAW_PHILOX,
                                 seed=philox_seed, step0=i * s2, max_survivors=1000)
        ms = timed(torch, stream, launch2, n2, warm=per) * n2
        tps = n2 * s2 * B / (ms / 1e3)
        ach = bytes_step * s2 * n2 / (ms / 1e3) / 1e9
        shapes["s%d" % s2] = {"steps_per_launch": s2, "tokens_per_s": round(tps, 1),
                              "hbm_frac": round(ach / HBM_PEAK_GBS, 5),
                              "ms_per_launch": round(ms / n2, 5)}

    # one launch per step: the decode-loop shape (launch latency included)
    single = None
    if args.single_launch_steps > 0:
        tok1 = torch.empty(B, dtype=torch.int32, device=dev)

        def one(i):
            sampler.sample_batch(slabs[i % args.slabs][(i % S) * B:(i % S + 1) * B], d_par, tok1,
                                 history=d_hist, history_len=d_hlen,
                                 draw_mode=mod.CBX_DRAW_PHILOX, seed=philox_seed, step0=i,
                                 max_survivors=1000)
        ms = timed(torch, stream, one, args.single_launch_steps, warm=10)
        single = {"ms_per_step": round(ms, 5), "tokens_per_s": round(B / (ms / 1e3), 1),
                  "latency_rows": 512 if args.latency_rows is None else args.latency_rows}

    # the decode loop with its state on the device, beside a per-token host sync
    decode = None
    if args.decode_steps > 0:
        decode = decode_loop_bench(torch, mod, sampler, dev, slabs, S, d_par, hist, hist_len,
                                   args.decode_steps, philox_seed)

    # the T3 transformer's decode step feeding the head and the sampler
    O = None
    if not args.no_cpu:
        import oracle_lib as O

    t3 = None
    if args.t3_steps > 0:
        # caches hold every timed position and the checked step after them
        n_ctx = max(512, 256 + args.t3_steps + 2)
        t3 = {"b64": t3_bench(torch, mod, sampler, dev, 64, 256, n_ctx, args.t3_steps, O),
              "b1": t3_bench(torch, mod, sampler, dev, 1, 256, n_ctx, args.t3_steps, O)}

    configs = None
    if not args.no_configs:
        configs = {"single_stream": config_single_stream(torch, mod, sampler, stream, dev, O),
                   "cfg_pair": config_cfg_pair(torch, mod, sampler, stream, dev, O),
                   "masked_stress": config_masked_stress(torch, mod, sampler, stream, dev)}

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
    if O is not None:
        # the last timed launch used this slab and these steps:
        last_slab = (n_launch_w + n_launch - 1) % args.slabs
        step0 = (n_launch_w + n_launch - 1) * S
        gpu_tokens = tokens.cpu().numpy()
        logits_host = slabs[last_slab].cpu().numpy()
        u = np.array([O.philox_uniform(philox_seed, r % B, step0 + r // B)
                      for r in range(S * B)])
        threads, visible = host_threads()
        res = cpu_baseline(O, hist, hist_len, params, logits_host, u, gpu_tokens,
                           args.cpu_seconds, args.cpu_mt_seconds, threads)
        import platform
        cpu = {"value": round(res["mt"][0], 1), "unit": "sampled tokens/s",
               "cores": threads, "kind": "port",
               "sample": "%d rows (B=256 streams x %d steps of the timed workload) on %d threads "
                         "(this GPU's share of the host; %d CPUs visible); single-thread: %.1f "
                         "tokens/s over %d rows; %s, %s" % (
                             res["mt"][1], res["mt"][1] // B, threads, visible, res["1t"][0],
                             res["1t"][1], cpu_model(), platform.machine()),
               "single_thread_value": round(res["1t"][0], 1)}
        parity = dict(rows_checked=res["rows_checked"], token_mismatches=res["mismatch"],
                      **res["classes"])

    out = {
        "metric": "sampled tokens/sec at B=256, V=6563; achieved HBM GB/s vs 8 TB/s peak",
        "value": round(tok_per_s, 1),
        "unit": "sampled tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": n_launch_w * S,
        "steps_requested": args.steps,
        "warmup_requested": args.warmup,
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
        "parity_vs_oracle": parity,
        "launch_shapes": shapes,
        "single_launch_per_step": single,
        "decode_loop": decode,
        "t3_decode": t3,
        "configs": configs,
        "fused_head": fused,
        "wall_s": round(time.perf_counter() - t_start, 1),
    }
    print(json.dumps(out), flush=True)
    sampler.close()


if __name__ == "__main__":
    main()

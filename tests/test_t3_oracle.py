"""Pins of the T3 decode-step oracle (oracle/cbx_t3_oracle.py) on the CPU,
against torch's own float64 routines: layer_norm, gelu(approximate="tanh"),
scaled_dot_product_attention, and a full-sequence causal forward written
with torch's functional ops (the prompt graph's form: every position at once
under a causal mask, main.cpp:490-497), which the oracle's position-by-
position decode with per-stream KV caches must reproduce.  A planted mistake
(k and v swapped in the fused projection) must fail that comparison.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
import torch.nn.functional as F  # noqa: E402

from oracle import cbx_t3_oracle as T3  # noqa: E402


def rand_model(rng, n_layer=2, n=256, H=4, n_pos=32, V=50, eps=1e-5):
    def w(o, i):
        return rng.standard_normal((o, i)) * 0.05

    def vec(k, base=0.0):
        return base + rng.standard_normal(k) * 0.1

    layers = [dict(ln_1_g=vec(n, 1.0), ln_1_b=vec(n), attn_w=w(3 * n, n), attn_b=vec(3 * n),
                   attn_proj_w=w(n, n), attn_proj_b=vec(n), ln_2_g=vec(n, 1.0), ln_2_b=vec(n),
                   fc_w=w(4 * n, n), fc_b=vec(4 * n), fc_proj_w=w(n, 4 * n), fc_proj_b=vec(n))
              for _ in range(n_layer)]
    return T3.Model(layers, rng.standard_normal((n_pos, n)) * 0.5,
                    rng.standard_normal((V, n)) * 0.5, vec(n, 1.0), vec(n), eps, H)


def torch_forward(m, xs):
    """Causal forward of one stream's input rows xs [T][n] with torch ops."""
    t = lambda a: torch.tensor(a, dtype=torch.float64)
    n, H = m.n_embd, m.n_head
    x = t(xs)
    T = x.shape[0]
    for L in m.layers:
        u = F.layer_norm(x, (n,), t(L["ln_1_g"]), t(L["ln_1_b"]), m.eps)
        q, k, v = F.linear(u, t(L["attn_w"]), t(L["attn_b"])).split(n, dim=1)
        heads = lambda z: z.reshape(T, H, T3.HEAD_DIM).transpose(0, 1)
        a = F.scaled_dot_product_attention(heads(q), heads(k), heads(v), is_causal=True)
        x = x + F.linear(a.transpose(0, 1).reshape(T, n), t(L["attn_proj_w"]),
                         t(L["attn_proj_b"]))
        u = F.layer_norm(x, (n,), t(L["ln_2_g"]), t(L["ln_2_b"]), m.eps)
        f = F.gelu(F.linear(u, t(L["fc_w"]), t(L["fc_b"])), approximate="tanh")
        x = x + F.linear(f, t(L["fc_proj_w"]), t(L["fc_proj_b"]))
    return F.layer_norm(x, (n,), t(m.ln_f_g), t(m.ln_f_b), m.eps).numpy()


def test_layer_norm_and_gelu_match_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 256)) * 3 + 1
    g, b = rng.standard_normal(256), rng.standard_normal(256)
    want = F.layer_norm(torch.tensor(x), (256,), torch.tensor(g), torch.tensor(b), 1e-5).numpy()
    assert np.allclose(T3.layer_norm(x, g, b, 1e-5), want, rtol=1e-12, atol=1e-12)
    y = np.linspace(-8, 8, 1001)
    assert np.allclose(T3.gelu(y), F.gelu(torch.tensor(y), approximate="tanh").numpy(),
                       rtol=1e-12, atol=1e-14)


def run_streams(m, seqs, skip=()):
    """Decode each stream's token sequence with the oracle, all streams per
    call; (stream, step) pairs in `skip` sit that call out.  Returns per
    stream the list of its ln_f rows."""
    R = len(seqs)
    kc, vc = T3.new_cache(R, len(m.layers), m.n_head, m.wpe.shape[0])
    pos = np.zeros(R, np.int64)
    done = [0] * R
    outs = [[] for _ in range(R)]
    call = 0
    while any(done[r] < len(seqs[r]) for r in range(R)):
        act = np.array([done[r] < len(seqs[r]) and (r, call) not in skip for r in range(R)])
        toks = np.array([seqs[r][min(done[r], len(seqs[r]) - 1)] for r in range(R)])
        out = T3.step(m, toks, pos, kc, vc, active=act)
        for r in np.nonzero(act)[0]:
            outs[r].append(out[r])
            done[r] += 1
        for r in np.nonzero(~act)[0]:
            assert np.all(out[r] == 0.0)
        call += 1
    assert list(pos) == [len(s) for s in seqs]
    return outs


def test_incremental_decode_equals_causal_forward():
    """Three streams of 5, 7 and 6 tokens, decoded together with some streams
    sitting some calls out (so their positions differ): every step's ln_f row
    equals the causal forward's row at that position."""
    rng = np.random.default_rng(2)
    m = rand_model(rng)
    seqs = [list(rng.integers(0, 50, L)) for L in (5, 7, 6)]
    outs = run_streams(m, seqs, skip={(0, 1), (2, 0), (2, 3), (1, 4)})
    for r, s in enumerate(seqs):
        xs = m.speech_emb[s] + m.wpe[:len(s)]
        want = torch_forward(m, xs)
        assert np.allclose(np.array(outs[r]), want, rtol=1e-10, atol=1e-10), r


def test_planted_kv_swap_fails():
    """The same comparison with k and v exchanged in the oracle's copy of the
    fused projection: the decode no longer reproduces the forward."""
    rng = np.random.default_rng(3)
    m = rand_model(rng)
    seq = list(rng.integers(0, 50, 4))
    want = torch_forward(m, m.speech_emb[seq] + m.wpe[:4])
    n = m.n_embd
    for L in m.layers:
        for key in ("attn_w", "attn_b"):
            a = L[key].copy()
            L[key][n:2 * n], L[key][2 * n:] = a[2 * n:], a[n:2 * n]
    got = np.array(run_streams(m, [seq])[0])
    assert not np.allclose(got[1:], want[1:], rtol=1e-6, atol=1e-6)


def test_prefill_equals_causal_forward():
    """The oracle's one-pass prompt (every row's k and v stored, then a causal
    mask) of a whole sequence from position 0 equals torch's causal
    forward."""
    rng = np.random.default_rng(4)
    m = rand_model(rng)
    seq = list(rng.integers(0, 50, 9))
    xs = m.speech_emb[seq] + m.wpe[:9]
    kc, vc = T3.new_cache(2, len(m.layers), m.n_head, m.wpe.shape[0])
    got = T3.prefill(m, xs, kc, vc, 1, 0)
    assert np.allclose(got, torch_forward(m, xs), rtol=1e-10, atol=1e-10)
    assert np.all(kc[0] == 0.0) and np.any(kc[1, :, :, 8] != 0.0)


def test_prefill_continues_a_cache():
    """A prompt continued from a cache the decode wrote (p0 = 6 positions
    decoded one at a time, then 5 more rows in one prefill pass) gives the
    rows the position-by-position decode gives, and leaves the same
    caches."""
    rng = np.random.default_rng(5)
    m = rand_model(rng)
    seq = list(rng.integers(0, 50, 11))
    kc, vc = T3.new_cache(1, len(m.layers), m.n_head, m.wpe.shape[0])
    kd, vd = T3.new_cache(1, len(m.layers), m.n_head, m.wpe.shape[0])
    pos, pd = np.zeros(1, np.int64), np.zeros(1, np.int64)
    want = []
    for t in range(11):
        out = T3.step(m, np.array([seq[t]]), pd, kd, vd)
        if t < 6:
            T3.step(m, np.array([seq[t]]), pos, kc, vc)
        else:
            want.append(out[0])
    xs = m.speech_emb[seq[6:]] + m.wpe[6:11]
    got = T3.prefill(m, xs, kc, vc, 0, 6)
    assert np.allclose(got, np.array(want), rtol=1e-10, atol=1e-10)
    assert np.allclose(kc[0, :, :, :11], kd[0, :, :, :11], rtol=0, atol=1e-12)
    assert np.allclose(vc[0, :, :, :11], vd[0, :, :, :11], rtol=0, atol=1e-12)


def test_stream_caches_index_like_dense():
    """Ragged per-stream caches (float32, as the reference's fp32 cache)
    give the step the dense binary64 cache gives, up to the fp32 rounding of
    the stored k and v."""
    rng = np.random.default_rng(7)
    m = rand_model(rng)
    nl, H = len(m.layers), m.n_head
    kd, vd = T3.new_cache(2, nl, H, m.wpe.shape[0])
    kr = T3.StreamCaches([np.zeros((nl, H, L, T3.HEAD_DIM), np.float32) for L in (5, 9)])
    vr = T3.StreamCaches([np.zeros((nl, H, L, T3.HEAD_DIM), np.float32) for L in (5, 9)])
    pd, pr = np.zeros(2, np.int64), np.zeros(2, np.int64)
    for t in range(5):
        toks = rng.integers(0, 50, 2)
        a = T3.step(m, toks, pd, kd, vd)
        b = T3.step(m, toks, pr, kr, vr)
        assert np.allclose(a, b, rtol=1e-5, atol=1e-5)
    # layer 0's first position: the same product, rounded once to fp32 (later
    # layers read the rounded v of earlier ones)
    assert np.array_equal(kr.arrays[1][0, :, 0], kd[1, 0, :, 0].astype(np.float32))
    assert np.allclose(kr.arrays[1][:, :, :5], kd[1, :, :, :5], rtol=1e-5, atol=1e-6)

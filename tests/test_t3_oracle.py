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

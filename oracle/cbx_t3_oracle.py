"""CPU oracle of the T3 transformer's decode step, in binary64 -- test
infrastructure only (imported by tests/ and nothing else; the product is
chatterbox.cpp_amd/csrc/cbx_t3.hip behind cbx_t3_step).

Restates the reference's GPT-2 core for N = 1 per stream (src/main.cpp:
469-575, step graph :617-633), many streams at once, each with its own KV
cache in the reference's per-layer [HD, n_ctx, n_head] order (stream
outermost: k[s][layer][head][pos][64]).  Matrices are given as float arrays
[n_out][n_in] (the format's values, dequantized exactly), so every product
here is exact-ish binary64.

Pinned (tests/test_t3_oracle.py) against torch's own routines on the CPU:
layer_norm, gelu(approximate="tanh") and scaled_dot_product_attention, and the
whole step, run position by position, against a full-sequence causal forward
written with torch's functional ops (the prompt graph's form, main.cpp:
490-497 mask).  `prefill` (one stream's prompt rows in one pass) is pinned
against that torch forward from position 0 and against the position-by-
position decode when it continues a cache; `StreamCaches` (ragged fp32
per-stream caches) against the dense binary64 cache.
"""
import numpy as np

HEAD_DIM = 64


def layer_norm(x, g, b, eps):
    """ggml_norm then mul and add (main.cpp:522-523): (x - mean) /
    sqrt(var + eps) * g + b, var the mean square of x - mean, per row."""
    x = np.asarray(x, np.float64)
    mean = x.mean(axis=-1, keepdims=True)
    d = x - mean
    var = (d * d).mean(axis=-1, keepdims=True)
    return d / np.sqrt(var + eps) * g + b


def gelu(x):
    """ggml_gelu's tanh form: 0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2)))."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * x * (1.0 + 0.044715 * x * x)))


class Model:
    """Binary64 copy of a cbx_t3_model: per layer dict of ln_1_g, ln_1_b,
    attn_w [3n][n], attn_b, attn_proj_w [n][n], attn_proj_b, ln_2_g, ln_2_b,
    fc_w [4n][n], fc_b, fc_proj_w [n][4n], fc_proj_b; wpe [n_pos][n],
    speech_emb [V][n], ln_f_g, ln_f_b, eps, n_head."""

    def __init__(self, layers, wpe, speech_emb, ln_f_g, ln_f_b, eps, n_head):
        f = lambda a: np.asarray(a, np.float64)
        # matrices keep their dtype: float32 values enter every product
        # exactly (numpy widens them to the binary64 operand's type)
        keep = lambda a: a if np.ndim(a) == 2 else f(a)
        self.layers = [{k: keep(v) for k, v in L.items()} for L in layers]
        self.wpe, self.speech_emb = f(wpe), f(speech_emb)
        self.ln_f_g, self.ln_f_b = f(ln_f_g), f(ln_f_b)
        self.eps, self.n_head = float(eps), int(n_head)
        self.n_embd = self.wpe.shape[1]


def new_cache(n_rows, n_layer, n_head, n_ctx):
    z = lambda: np.zeros((n_rows, n_layer, n_head, n_ctx, HEAD_DIM), np.float64)
    return z(), z()


def step(m, tokens, positions, kc, vc, inputs=None, active=None):
    """One decode step (main.cpp:617-633 + :469-575 with N = 1) of every
    active stream r: input speech_emb[tokens[r]] + wpe[positions[r]] (or
    inputs[r]), k and v appended at positions[r], attention over [0, pos].
    Updates kc, vc and positions in place; returns ln_f rows [n_rows][n]
    (zero for inactive rows)."""
    n, H = m.n_embd, m.n_head
    R = len(positions)
    active = np.ones(R, bool) if active is None else np.asarray(active, bool)
    x = np.zeros((R, n))
    for r in np.nonzero(active)[0]:
        x[r] = (np.asarray(inputs[r], np.float64) if inputs is not None
                else m.speech_emb[tokens[r]] + m.wpe[positions[r]])
    for li, L in enumerate(m.layers):
        u = layer_norm(x, L["ln_1_g"], L["ln_1_b"], m.eps)
        qkv = u @ L["attn_w"].T + L["attn_b"]
        att = np.zeros((R, n))
        for r in np.nonzero(active)[0]:
            p = int(positions[r])
            for h in range(H):
                sl = slice(h * HEAD_DIM, (h + 1) * HEAD_DIM)
                q = qkv[r, sl]
                kc[r, li, h, p] = qkv[r, n:][sl]
                vc[r, li, h, p] = qkv[r, 2 * n:][sl]
                s = kc[r, li, h, :p + 1] @ q / np.sqrt(HEAD_DIM)
                w = np.exp(s - s.max())
                att[r, sl] = (w / w.sum()) @ vc[r, li, h, :p + 1]
        x = x + att @ L["attn_proj_w"].T + L["attn_proj_b"]
        u = layer_norm(x, L["ln_2_g"], L["ln_2_b"], m.eps)
        f = gelu(u @ L["fc_w"].T + L["fc_b"])
        x = x + f @ L["fc_proj_w"].T + L["fc_proj_b"]
    out = layer_norm(x, m.ln_f_g, m.ln_f_b, m.eps)
    out[~active] = 0.0
    for r in np.nonzero(active)[0]:
        positions[r] += 1
    return out


class StreamCaches:
    """Per-stream caches of different lengths, indexed like new_cache's
    arrays (c[r, layer, head, pos], c[r, layer, head, :p + 1]): stream r's
    array is arrays[r] [n_layer][n_head][n_r][64], any float dtype (float32
    stores what the reference's fp32 cache holds).  For long contexts where
    one dense [n_rows][...][n_ctx][64] binary64 array would not fit."""

    def __init__(self, arrays):
        self.arrays = list(arrays)

    def __getitem__(self, key):
        return self.arrays[key[0]][tuple(key[1:])]

    def __setitem__(self, key, value):
        self.arrays[key[0]][tuple(key[1:])] = value


def prefill(m, inputs, kc, vc, slot, p0):
    """One stream's prompt rows at positions p0 .. p0 + T - 1 in one pass (the
    prompt graph, main.cpp:643-689 up to ln_f, with n_past = p0): inputs
    [T][n] embedded rows; every row's k and v stored in cache slot `slot`
    before any row attends, row t attending over [0, p0 + t] (the causal mask
    of main.cpp:490-497; positions below p0 are read from the cache as they
    stand).  Returns the rows' ln_f outputs [T][n]."""
    n, H = m.n_embd, m.n_head
    x = np.asarray(inputs, np.float64).copy()
    T = x.shape[0]
    end = p0 + T
    # row t may not see position j > p0 + t
    mask = np.arange(end)[None, :] > (p0 + np.arange(T))[:, None]
    for li, L in enumerate(m.layers):
        u = layer_norm(x, L["ln_1_g"], L["ln_1_b"], m.eps)
        qkv = u @ L["attn_w"].T + L["attn_b"]
        att = np.zeros((T, n))
        for h in range(H):
            sl = slice(h * HEAD_DIM, (h + 1) * HEAD_DIM)
            kc[slot, li, h, p0:end] = qkv[:, n:][:, sl]
            vc[slot, li, h, p0:end] = qkv[:, 2 * n:][:, sl]
            K = np.asarray(kc[slot, li, h, :end], np.float64)
            V = np.asarray(vc[slot, li, h, :end], np.float64)
            s = qkv[:, sl] @ K.T / np.sqrt(HEAD_DIM)
            s[mask] = -np.inf
            w = np.exp(s - s.max(axis=1, keepdims=True))
            att[:, sl] = (w / w.sum(axis=1, keepdims=True)) @ V
        x = x + att @ L["attn_proj_w"].T + L["attn_proj_b"]
        u = layer_norm(x, L["ln_2_g"], L["ln_2_b"], m.eps)
        f = gelu(u @ L["fc_w"].T + L["fc_b"])
        x = x + f @ L["fc_proj_w"].T + L["fc_proj_b"]
    return layer_norm(x, m.ln_f_g, m.ln_f_b, m.eps)

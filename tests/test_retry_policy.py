"""cbx_retry_* (include/cbx_retry.h, chatterbox.cpp_amd/csrc/cbx_retry.cpp):
the T3 segment loop's early-stop retry policy, src/chatterbox_cli.cpp:1614-1672.

Each scenario below is a sequence of attempt outcomes (speech tokens after
popping the stop token, ended on the stop token or not) with the attempt the
reference keeps, worked out from that loop by hand: it breaks on the first
attempt that did not end on the stop token or reached min_tokens =
max(8, 5 * text tokens); after MAX_RETRIES = 3 retries it keeps
best_generated, which only a strictly longer attempt replaces.  CPU only.
"""
import numpy as np
import pytest

import oracle_lib as O
import pkg

U64_MAX = (1 << 64) - 1


@pytest.fixture(scope="module")
def mod():
    return pkg.load()


def run(mod, n_text, outcomes):
    r = mod.retry_start(n_text)
    ran = []
    for n, stopped in outcomes:
        ran.append(r.attempt)
        if not mod.retry_record(r, n, stopped):
            break
    return r, ran


@pytest.mark.parametrize("n_text,min_tokens", [(0, 8), (1, 8), (2, 10), (40, 200)])
def test_min_tokens(mod, n_text, min_tokens):
    assert mod.retry_start(n_text).min_tokens == min_tokens


SCENARIOS = [
    # n_text, outcomes, attempts run, kept attempt, kept length
    (4, [(3, False)], [0], 0, 3),                      # n_predict reached: kept even if short
    (4, [(20, True)], [0], 0, 20),                     # stop token, long enough
    (4, [(19, True), (20, True)], [0, 1], 1, 20),      # 19 < 20 = min_tokens: one retry
    (4, [(5, True), (6, True), (30, False)], [0, 1, 2], 2, 30),
    (4, [(3, True), (7, True), (7, True), (5, True)], [0, 1, 2, 3], 1, 7),   # first of the longest
    (0, [(0, True)] * 4, [0, 1, 2, 3], 0, 0),
    (1, [(7, True), (8, True)], [0, 1], 1, 8),         # floor of 8 tokens
    (2, [(1, True), (2, True), (3, True), (9, True)], [0, 1, 2, 3], 3, 9),
]


@pytest.mark.parametrize("n_text,outcomes,ran,kept,kept_len", SCENARIOS)
def test_scenarios(mod, n_text, outcomes, ran, kept, kept_len):
    r, got_ran = run(mod, n_text, outcomes)
    assert got_ran == ran
    assert r.done == 1 and (r.kept_attempt, r.kept_len) == (kept, kept_len)


def test_errors(mod):
    r, _ = run(mod, 4, [(30, True)])
    with pytest.raises(mod.CbxError):
        mod.retry_record(r, 1, True)           # after done
    with pytest.raises(mod.CbxError):
        mod.retry_start(-1)
    r = mod.retry_start(1)
    with pytest.raises(mod.CbxError):
        mod.retry_record(r, -1, True)


def test_stream_ids(mod):
    assert mod.retry_stream_id(0, 0) == 0 and mod.retry_stream_id(6562, 0) == 6562
    ids = {mod.retry_stream_id(s, a) for s in list(range(300)) + [(1 << 56) - 1] for a in range(4)}
    assert len(ids) == 301 * 4
    assert mod.retry_stream_id(1 << 56, 0) == U64_MAX
    assert mod.retry_stream_id(5, 4) == U64_MAX and mod.retry_stream_id(5, -1) == U64_MAX
    # the attempts of a stream draw different uniforms (oracle Philox)
    seqs = [tuple(O.philox_uniform(42, mod.retry_stream_id(7, a), t) for t in range(16))
            for a in range(4)]
    assert len(set(seqs)) == 4
    assert all(0.0 <= u < 1.0 for s in seqs for u in s)


STOP = 6562


def loop_reference(draws, n_predict, stop=STOP, n_ctx_left=None):
    """The decode loop of chatterbox_cli.cpp:1627-1648 over a fixed sequence
    of draws: (tokens kept after the pop, stopped_by_stop_token, tokens drawn)."""
    it = iter(draws)
    current = next(it)
    generated = [current]
    stopped = False
    for i in range(n_predict):
        if current == stop:
            stopped = True
            break
        if n_ctx_left is not None and i >= n_ctx_left:
            break  # "KV cache full"
        current = next(it)
        generated.append(current)
    n_drawn = len(generated)
    if generated and generated[-1] == stop:
        generated.pop()
    return len(generated), stopped, n_drawn


@pytest.mark.parametrize("draws,n_predict,n_ctx_left", [
    ([1, 2, 3, STOP], 10, None),          # stop drawn early: stopped, retried when short
    ([1] * 10 + [STOP], 10, None),        # stop drawn by the last iteration: not stopped
    ([1] * 11, 10, None),                 # n_predict ran out
    ([STOP], 0, None),                    # n_predict 0: the prompt's token only
    ([STOP], 5, None),                    # the prompt's token is the stop token
    ([1, 2, 3, 4, 5], 10, 3),             # context full after 3 iterations
])
def test_record_tokens_matches_the_loop(mod, draws, n_predict, n_ctx_left):
    """cbx_retry_record_tokens derives the reference loop's flag and length
    from the tokens drawn, including a stop token drawn by the last of the
    n_predict iterations (popped, but the attempt counts as not stopped)."""
    n_tok, stopped, n_drawn = loop_reference(draws, n_predict, n_ctx_left=n_ctx_left)
    last = draws[n_drawn - 1]
    a = mod.retry_start(4)     # min_tokens 20: every attempt here is short
    b = mod.retry_start(4)
    again_a = mod.retry_record(a, n_tok, stopped)
    again_b = mod.retry_record_tokens(b, n_drawn, last, STOP, n_predict)
    assert again_a == again_b == stopped
    assert (a.best_len, a.attempt, a.done) == (b.best_len, b.attempt, b.done)


def test_stop_on_last_iteration_is_kept(mod):
    """A 10-token attempt whose 11th draw (by iteration n_predict - 1) is the
    stop token is kept although it is shorter than min_tokens: the reference
    never sets stopped_by_stop_token for it."""
    r = mod.retry_start(4)
    assert not mod.retry_record_tokens(r, 11, STOP, STOP, 10)
    assert r.done == 1 and (r.kept_attempt, r.kept_len) == (0, 10)
    r = mod.retry_start(4)
    assert mod.retry_record_tokens(r, 10, STOP, STOP, 10)  # drawn by iteration 8: retried
    assert r.attempt == 1 and r.best_len == 9


def test_record_tokens_rejects_impossible_counts(mod):
    r = mod.retry_start(1)
    for n_sampled, n_predict in ((0, 5), (7, 5), (1, -1)):
        with pytest.raises(mod.CbxError):
            mod.retry_record_tokens(r, n_sampled, 1, STOP, n_predict)

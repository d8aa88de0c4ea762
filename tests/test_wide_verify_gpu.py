"""Verify lists of 9..64 rows (the reference's wide and deep lists: control.h:35-42 for their
id slots, verify_attn.h:65-92 for the attention they bind). The engine runs such a list in
row chunks of 8 with the attention over all rows at once. Where the decode kernel serves the
attention, every row must be bitwise the same row of a plain single-row step (property R of
the GEMV, attn_prep and the decode kernel); where the rule binds the many-row verify kernel
(16 / 2 heads of 256 at 16, 32, 64 rows), the rows are held to the fp64-checked kernel's bar
against the plain steps' logits, with every argmax equal or a near-tie."""
import numpy as np
import pytest

from mipkg import mi
from test_engine_gpu import argmax_ok, close, moe_small_desc, small_desc

pytestmark = pytest.mark.gpu


def plain_steps(eng, P, t0, n):
    """n single-row greedy steps from (P, t0): the tokens and each step's logits"""
    eng.reset(P, t0)
    toks, lg = [], []
    for _ in range(n):
        toks.append(int(eng.generate(1)[0]))
        lg.append(eng.logits(1)[0].copy())
    return toks, lg


def slots(M):
    return (mi.CTRL_CUR, mi.CTRL_OUT) if M <= 8 else \
        (mi.CTRL_WIDE_CUR, mi.CTRL_WIDE_OUT) if M <= 16 else (mi.CTRL_DEEP_CUR, mi.CTRL_DEEP_OUT)


@pytest.mark.parametrize("kw,k,seed", [
    (dict(), 11, 31),                       # 12 rows: a chunk of 8 and one of 4 (q||k||v with attn_prep fused)
    (dict(), 15, 32),                       # 16 rows at 8 / 2 heads of 128: the decode kernel per chunk
    (dict(), 40, 33),                       # 41 rows: the deep slots, a ragged last chunk
    (dict(head_dim=256, kv_int8=1), 19, 34),   # the int8 cache's writer and reader per chunk
    (dict(lm_head_int8=1), 9, 35),          # the int8 head per chunk
    (dict(act_bf16=1), 13, 36),             # bf16 activations
])
def test_wide_rows_bitwise_plain_steps(kw, k, seed):
    M = k + 1
    print(f"wide verify {kw} rows {M}", flush=True)
    eng = mi.Engine(small_desc(max_rows=64, **kw), seed=seed)
    eng.capture(1)
    P, t0 = 90, 7
    toks, lg = plain_steps(eng, P, t0, M)
    eng.reset(P, t0)
    rows = eng.verify(toks[:k])
    assert list(rows) == toks
    c = eng.ctrl()
    cur, out = slots(M)
    assert list(c[out:out + M]) == toks and list(c[cur:cur + M]) == [t0] + toks[:k]
    assert c[mi.CTRL_POS] == P and c[mi.CTRL_DEBUG] == 0
    got = eng.logits(M)
    for m in range(M):
        assert np.array_equal(got[m].view(np.uint32), lg[m].view(np.uint32)), m
    # accept everything, commit, and continue plainly: the next token is the plain run's
    j, nxt = mi.accept_greedy(rows, toks[:k])
    assert (j, nxt) == (k, toks[k])
    eng.commit(P, j, nxt)
    assert eng.ctrl()[mi.CTRL_POS] == P + M
    eng.close()


def test_wide_moe_rows_bitwise_plain_steps():
    M = 10
    eng = mi.Engine(moe_small_desc(max_rows=16), seed=37)
    eng.capture(1)
    P, t0 = 40, 5
    toks, lg = plain_steps(eng, P, t0, M)
    eng.reset(P, t0)
    rows = eng.verify(toks[:M - 1])
    assert list(rows) == toks
    got = eng.logits(M)
    for m in range(M):
        assert np.array_equal(got[m].view(np.uint32), lg[m].view(np.uint32)), m
    eng.close()


@pytest.mark.parametrize("M", [16, 32, 64])
def test_wide_rows_bind_the_verify_kernel(M):
    """16 / 2 heads of 256: the rule binds the many-row kernel at 16, 32 and 64 rows. Its
    partials come from a different walk than the decode kernel's, so the rows are held to the
    logit bar of the engine tests against the plain steps, with every argmax equal or an
    oracle-style near-tie, and a rejected draft stops the accept where the plain run differs."""
    assert mi.lib().mi_attn_verify_binds(M, 0, 16, 2) == 1
    eng = mi.Engine(small_desc(q_heads=16, kv_heads=2, head_dim=256, max_rows=64, max_len=1024), seed=40 + M)
    eng.capture(1)
    P, t0 = 300, 11
    toks, lg = plain_steps(eng, P, t0, M)
    eng.reset(P, t0)
    rows = eng.verify(toks[:M - 1])
    got = eng.logits(M)
    for m in range(M):
        assert close(got[m], lg[m], abs_frac=1e-3), m
        assert argmax_ok(int(rows[m]), lg[m], abs_frac=1e-3), m
    j, nxt = mi.accept_greedy(rows, toks[:M - 1])
    assert j <= M - 1
    eng.commit(P, j, nxt)
    assert eng.ctrl()[mi.CTRL_POS] == P + j + 1
    eng.close()


def test_wide_refusals():
    # more than 64 rows, and an MTP head with more than 8
    for kw in (dict(max_rows=65), dict(max_rows=9, mtp=1)):
        d = small_desc(**kw)
        assert not mi.lib().mi_engine_create(mi.C.byref(d), 1, None)
    eng = mi.Engine(small_desc(max_rows=12), seed=1)
    eng.capture(1)
    eng.reset(20, 3)
    with pytest.raises(mi.MiError):
        eng.verify(list(range(12)))  # 13 rows > max_rows
    eng.close()

"""The MTP head's draft lists and K/V fill on the GPU (capture.cc:1772-1939, 362-370;
Engine::draft / verify / commit, engine.h:259-290) against the oracle's head
(orc_mtp_head_step, pinned by an fp64 forward in test_oracle_step.py).

Bars: each draft's id is the oracle's argmax on the same inputs (the previous draft's id and
the head's own hidden) unless the oracle's top two are within the logits tolerance; the last
draft's logits, the head's K/V rows and the chained hidden within rel 2e-3 of the oracle's
(plus 2e-3 of the row's largest value); commit
moves the accepted row's hidden bitwise; a speculative loop (draft, verify, accept_greedy,
commit) emits exactly the plain greedy tokens."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import mi
from test_engine_gpu import OracleModel, argmax_ok, close, moe_small_desc, small_desc

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16


class OracleHead:
    """Host copies of the engine's MTP head wired into orc_mtp_head."""

    def __init__(self, eng, orc):
        d = eng.desc
        self.eng, self.orc, self.d = eng, orc, d
        H, HD, QH, KVH, I = d.hidden, d.head_dim, d.q_heads, d.kv_heads, d.inter
        keep = self.keep = []

        def h(a):
            a = np.ascontiguousarray(a)
            keep.append(a)
            return a

        li = d.layers
        moe = d.experts > 0
        w16 = bool(d.mtp_w16)  # the 16-bit head: its f16 tiles, the int4 fields unused
        S = [eng.linear_s(w) for w in range(4)]
        lins = []
        for w, (K, N) in enumerate([(H, (QH + 2 * KVH) * HD), (QH * HD, H), (H, 2 * I), (I, H)]):
            if (moe and w >= 2) or w16:  # an MoE model's head: its MoE layer instead of gate||up / down
                lins.append(O.Linear(None, None, K, N, 1))
                continue
            q = h(eng.to_host(2 * w, li, np.uint32))
            s = h(eng.to_host(2 * w + 1, li, np.uint16))
            lins.append(O.Linear(q.ctypes.data, s.ctypes.data, K, N, S[w]))
        L = O.Layer()
        L.qkv, L.o, L.gate_up, L.down = lins
        if moe:
            L.router = h(eng.to_host(mi.T_ROUTER, li, np.uint16)).ctypes.data
            L.moe_gu = h(eng.to_host(mi.T_MOE_GU, li, np.uint32)).ctypes.data
            L.moe_dn = h(eng.to_host(mi.T_MOE_DN, li, np.uint32)).ctypes.data
        L.in_norm = h(eng.to_host(mi.T_IN_NORM, li, np.float32)).ctypes.data
        L.post_norm = h(eng.to_host(mi.T_POST_NORM, li, np.float32)).ctypes.data
        if d.qk_norm:
            L.q_norm = h(eng.to_host(mi.T_Q_NORM, li, np.float32)).ctypes.data
            L.k_norm = h(eng.to_host(mi.T_K_NORM, li, np.float32)).ctypes.data
        pe = h(eng.to_host(mi.T_MTP_PRE_E, 0, np.float32))
        ph = h(eng.to_host(mi.T_MTP_PRE_H, 0, np.float32))
        fn = h(eng.to_host(mi.T_MTP_FINAL, 0, np.float32))
        if w16:
            fc = O.Linear(None, None, 0, 0, 0)
            w16s = [h(eng.to_host(k, 0, np.uint16)).ctypes.data for k in
                    (mi.T_MTP_W16_FC, mi.T_MTP_W16_QKV, mi.T_MTP_W16_O, mi.T_MTP_W16_GU, mi.T_MTP_W16_DN)]
        else:
            fcq = h(eng.to_host(mi.T_MTP_FC_Q, 0, np.uint32))
            fcs = h(eng.to_host(mi.T_MTP_FC_S, 0, np.uint16))
            fc = O.Linear(fcq.ctypes.data, fcs.ctypes.data, 2 * H, H, eng.linear_s(5))
            w16s = []
        self.head = O.MtpHead(fc, L, pe.ctypes.data, ph.ctypes.data, fn.ctypes.data, *w16s)
        keep.append(L)

    def run(self, tok, h16, p, kk, vv, full=1):
        logits = np.zeros(self.d.vocab, np.float32)
        hout = np.zeros(self.d.hidden, np.uint16)
        am = O.lib().orc_mtp_head_step(F16, C.byref(self.orc.m), C.byref(self.head), int(tok), O._p(h16), int(p),
                                       O._p(kk), O._p(vv), full, O._p(hout), O._p(logits))
        return int(am), logits, hout


def f16_close(got, want, ulps=None):
    """fp16 rows within the logits bar: rel 2e-3 of each value plus 2e-3 of the row's largest
    (the head's rows come from fp32 sums in another order, rounded once, and a chained draft
    feeds its hidden to the next)."""
    g = O.f16_bits_to_f32(got).astype(np.float64)
    w = O.f16_bits_to_f32(want).astype(np.float64)
    tol = 2e-3 * np.abs(w) + 2e-3 * np.abs(w).max(axis=-1, keepdims=True)
    return np.all(np.abs(g - w) <= tol), np.abs(g - w).max()


def head_kv(eng):
    return eng.to_host(mi.T_MTP_KV_K, 0, np.uint16).reshape(eng.desc.kv_heads, eng.desc.max_len, -1).copy(), \
        eng.to_host(mi.T_MTP_KV_V, 0, np.uint16).reshape(eng.desc.kv_heads, eng.desc.max_len, -1).copy()


def make(seed=42, moe=False, **kw):
    eng = mi.Engine((moe_small_desc if moe else small_desc)(mtp=1, **kw), seed=seed)
    orc = OracleModel(eng)
    return eng, orc, OracleHead(eng, orc)


@pytest.mark.parametrize("kind", ["dense", "kv8", "moe", "w16"])
def test_drafts_vs_oracle_head_chain(kind):
    # kv8: the main model over the int8 rotated cache (head_dim 256); the head keeps its own f16
    # cache. moe: an MoE model, whose head is one MoE layer (spec 15e). w16: the dense head's
    # linears in 16 bits (the reference's bf16 head, loader.cc:586-597)
    eng, orc, oh = make(**{"dense": {}, "kv8": dict(head_dim=256, kv_int8=1), "moe": dict(moe=True),
                           "w16": dict(mtp_w16=1)}[kind])
    H = eng.desc.hidden
    eng.capture(1)
    eng.reset(300, 7)
    eng.generate(3)  # the steps fill the head's K/V and leave h_{pos-1} in hh row 0
    c = eng.ctrl()
    pos, cur = int(c[mi.CTRL_POS]), int(c[mi.CTRL_CUR])
    hh0 = eng.to_host(mi.T_MTP_HH, 0, np.uint16)[:H].copy()
    kk, vv = head_kv(eng)
    print(f"mtp drafts at pos {pos} cur {cur}", flush=True)
    drafts = eng.draft(3)
    gk, gv = head_kv(eng)
    tok, h = cur, hh0
    for i in range(3):
        am, logits, hout = oh.run(tok, h, pos - 1 + i, kk, vv)
        assert argmax_ok(int(drafts[i]), logits), (i, drafts[i], am)
        tok, h = int(drafts[i]), hout  # teacher-forced on the GPU's ids, the oracle's own hidden
    got = eng.to_host(mi.T_MTP_LOGITS, 0, np.float32)
    assert close(got, logits), np.abs(got - logits).max()
    ok, err = f16_close(eng.to_host(mi.T_MTP_DH, 0, np.uint16), h, ulps=8)
    assert ok, err
    for p in range(pos - 1, pos + 2):  # the rows the three draft lists wrote
        for a, b in ((gk, kk), (gv, vv)):
            ok, err = f16_close(a[:, p], b[:, p], ulps=8)
            assert ok, (p, err)
    mask = np.ones(eng.desc.max_len, bool)
    mask[pos - 1:pos + 2] = False
    assert np.array_equal(gk[:, mask], kk[:, mask]) and np.array_equal(gv[:, mask], vv[:, mask])
    assert eng.ctrl()[mi.CTRL_POS] == pos  # the main model's state is untouched


@pytest.mark.parametrize("w16", [0, 1])
def test_verify_fills_the_head_and_commit_moves_the_hidden(w16):
    eng, orc, oh = make(seed=5, mtp_w16=w16)
    H = eng.desc.hidden
    eng.capture(1)
    eng.reset(200, 11)
    eng.generate(2)
    c = eng.ctrl()
    pos, cur = int(c[mi.CTRL_POS]), int(c[mi.CTRL_CUR])
    drafts = eng.draft(3)
    kk, vv = head_kv(eng)
    print(f"mtp verify at pos {pos} drafts {list(drafts)}", flush=True)
    am = eng.verify(drafts)
    hh = eng.to_host(mi.T_MTP_HH, 0, np.uint16).reshape(-1, H).copy()
    # the fill: hh rows 0..3 with the rows' ids [cur, d1, d2, d3] at pos - 1 .. pos + 2
    ids = [cur] + [int(t) for t in drafts]
    gk, gv = head_kv(eng)
    for r in range(4):
        oh.run(ids[r], hh[r], pos - 1 + r, kk, vv, full=0)
        for a, b in ((gk, kk), (gv, vv)):
            ok, err = f16_close(a[:, pos - 1 + r], b[:, pos - 1 + r], ulps=8)
            assert ok, (r, err)
    j, nxt = mi.accept_greedy(am, drafts)
    eng.commit(pos, j, nxt)
    hh2 = eng.to_host(mi.T_MTP_HH, 0, np.uint16).reshape(-1, H)
    assert np.array_equal(hh2[0], hh[j + 1])
    c2 = eng.ctrl()
    assert c2[mi.CTRL_POS] == pos + j + 1 and c2[mi.CTRL_CUR] == nxt


def test_plain_steps_keep_the_head_filled():
    """generate's step (verify(0) + commit(0)): each step fills the head's row at pos - 1 from
    (hh row 0, the step's id) and leaves its own hidden in hh row 0."""
    eng, orc, oh = make(seed=9)
    H = eng.desc.hidden
    eng.capture(1)
    eng.reset(0, 3)
    for s in range(4):
        c = eng.ctrl()
        pos, cur = int(c[mi.CTRL_POS]), int(c[mi.CTRL_CUR])
        hh0 = eng.to_host(mi.T_MTP_HH, 0, np.uint16)[:H].copy()
        kk, vv = head_kv(eng)
        print(f"mtp plain step {s} pos {pos}", flush=True)
        eng.generate(1)
        gk, gv = head_kv(eng)
        if pos == 0:  # no h_{-1}: nothing filled
            assert np.array_equal(gk, kk) and np.array_equal(gv, vv)
        else:
            oh.run(cur, hh0, pos - 1, kk, vv, full=0)
            for a, b in ((gk, kk), (gv, vv)):
                ok, err = f16_close(a[:, pos - 1], b[:, pos - 1], ulps=8)
                assert ok, (s, err)
        hh = eng.to_host(mi.T_MTP_HH, 0, np.uint16).reshape(-1, H)
        assert np.array_equal(hh[0], hh[1])  # committed at once


@pytest.mark.parametrize("moe", [False, True])
def test_prefill_fills_the_head_like_ingest(moe):
    """step_mtp_kv: a prefilled prompt leaves the head's K/V rows 0..n-2 and hh row 0 within the
    prefill's bar of the token-by-token ingest's (the prefill's hidden rows carry its own
    roundings: rel 2e-2 of the rows' largest value); also on an MoE model."""
    ids = np.random.default_rng(4).integers(0, 4096, 40).astype(np.uint32)
    outs = []
    for way in ("prefill", "ingest"):
        eng = mi.Engine((moe_small_desc if moe else small_desc)(mtp=1, max_rows=4), seed=77)
        eng.capture(1)
        eng.reset(0, int(ids[0]))
        print(f"mtp {way} of {ids.size} ids", flush=True)
        if way == "prefill":
            eng.prefill(ids, chunk=16)
        else:
            eng.ingest(ids)
        hk, hv = head_kv(eng)
        outs.append((hk, hv, eng.to_host(mi.T_MTP_HH, 0, np.uint16)[:eng.desc.hidden].copy(), eng.ctrl()))
    (pk, pv, ph, pc), (ik, iv, ih, ic) = outs
    assert pc[mi.CTRL_POS] == ic[mi.CTRL_POS] == ids.size
    n = ids.size - 1
    for a, b in ((pk[:, :n], ik[:, :n]), (pv[:, :n], iv[:, :n]), (ph, ih)):
        x = O.f16_bits_to_f32(a).astype(np.float64)
        y = O.f16_bits_to_f32(b).astype(np.float64)
        assert np.abs(x - y).max() <= 2e-2 * np.abs(y).max(), np.abs(x - y).max()


@pytest.mark.parametrize("kind", ["dense", "kv8", "moe", "w16"])
def test_speculative_loop_emits_the_greedy_tokens(kind):
    """draft(3) -> verify -> accept_greedy -> commit, repeated, against plain generate on a twin
    engine: the same token stream, bit for bit (verify rows are bitwise the plain steps); also
    with the main model over the int8 cache, and with the 16-bit head."""
    n = 14
    kw = dict(head_dim=256, kv_int8=1) if kind == "kv8" else dict(mtp_w16=1) if kind == "w16" else {}
    mk = moe_small_desc if kind == "moe" else small_desc
    plain = mi.Engine(mk(mtp=1, **kw), seed=31)
    plain.capture(1)
    plain.reset(100, 5)
    want = list(plain.generate(n))
    eng = mi.Engine(mk(mtp=1, **kw), seed=31)
    eng.capture(1)
    eng.reset(100, 5)
    got, accepted = [], 0
    first = eng.generate(1)  # pos 100 -> 101, so the head has h_{pos-1}
    got.append(int(first[0]))
    while len(got) < n:
        c = eng.ctrl()
        pos = int(c[mi.CTRL_POS])
        drafts = eng.draft(3)
        am = eng.verify(drafts)
        j, nxt = mi.accept_greedy(am, drafts)
        accepted += j
        got += [int(t) for t in drafts[:j]] + [int(nxt)]
        eng.commit(pos, j, nxt)
    print(f"speculative: {accepted} drafts accepted over {len(got)} tokens", flush=True)
    assert got[:n] == want

"""Loading a synthetic GPTQ / AutoRound checkpoint into an engine on the GPU (mi_engine_load):
every device tensor against the layout its format defines, computed here from the
checkpoint's arrays (q||k||v by columns; gate/up interleaved in 16-column blocks with the
oracle's repack.h restatement; experts as layout-1 tiles; the router as f16 tiles; norms fp32;
embeddings f16), the int4 head quantised at load within half a scale step, and a decode step
of the loaded model against the CPU oracle's step on the same weights."""
import numpy as np
import pytest

import oracle as O
from ckpt_synth import Synth
from mipkg import mi
from test_engine_gpu import OracleModel, argmax_ok, close

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16


def expect_interleave(a, b):
    """repack.h interleave16 of two [rows][Np] arrays (column n: a's (n/32)16 + n%16 when
    n % 32 < 16, else b's)"""
    rows, Np = a.shape
    n = np.arange(2 * Np)
    src = (n // 32) * 16 + n % 16
    return np.where((n % 32 < 16)[None, :], a[:, src], b[:, src])


def load(syn, max_len=512, max_rows=4):
    path = syn.write(split=2)
    desc = mi.checkpoint_desc(path, max_len=max_len, max_rows=max_rows)
    eng = mi.Engine(desc, seed=5)
    print(f"engine_load {path}: {eng.load(path)}", flush=True)
    return eng


def test_dense_tensors_and_step(tmp_path):
    syn = Synth(str(tmp_path / "d"), V=4000)
    eng = load(syn)
    d = eng.desc
    H, I, Vp = d.hidden, d.inter, d.vocab
    for li, L in enumerate(syn.layers):
        qkv_q = np.concatenate([L["q"][0], L["k"][0], L["v"][0]], axis=1)
        qkv_s = np.concatenate([L["q"][1], L["k"][1], L["v"][1]], axis=1)
        assert np.array_equal(eng.to_host(mi.T_QKV_Q, li, np.uint32), qkv_q.ravel())
        assert np.array_equal(eng.to_host(mi.T_QKV_S, li, np.uint16), qkv_s.ravel())
        assert np.array_equal(eng.to_host(mi.T_O_Q, li, np.uint32), L["o"][0].ravel())
        assert np.array_equal(eng.to_host(mi.T_O_S, li, np.uint16), L["o"][1].ravel())
        gu_q = expect_interleave(L["gate"][0], L["up"][0])
        gu_s = expect_interleave(L["gate"][1], L["up"][1])
        # the same map as the oracle's repack.h restatement (itself pinned by the reference's twin)
        oq = np.empty(gu_q.size, np.uint32)
        os_ = np.empty(gu_s.size, np.uint16)
        O.lib().orc_interleave16_l0(O._p(L["gate"][0]), O._p(L["gate"][1]), O._p(L["up"][0]), O._p(L["up"][1]),
                                    H, I, O._p(oq), O._p(os_))
        assert np.array_equal(oq, gu_q.ravel()) and np.array_equal(os_, gu_s.ravel())
        assert np.array_equal(eng.to_host(mi.T_GU_Q, li, np.uint32), gu_q.ravel())
        assert np.array_equal(eng.to_host(mi.T_GU_S, li, np.uint16), gu_s.ravel())
        assert np.array_equal(eng.to_host(mi.T_DOWN_Q, li, np.uint32), L["down"][0].ravel())
        for kind, key in ((mi.T_IN_NORM, "in_norm"), (mi.T_POST_NORM, "post_norm"), (mi.T_Q_NORM, "q_norm"),
                          (mi.T_K_NORM, "k_norm")):
            assert np.array_equal(eng.to_host(kind, li, np.float32), L[key].astype(np.float32)), key
    emb = eng.to_host(mi.T_EMBED, 0, np.uint16).reshape(Vp, H)
    assert np.array_equal(emb[:syn.d["V"]], O.f32_to_f16_bits(syn.embed))
    assert not emb[syn.d["V"]:].any()
    lmq = eng.to_host(mi.T_LM_Q, 0, np.uint32).reshape(H // 8, Vp)
    assert np.array_equal(lmq[:, :syn.d["V"]], syn.lm[0])
    assert np.array_equal(eng.to_host(mi.T_FINAL_NORM, 0, np.float32), syn.final_norm)
    # a decode step of the loaded model against the oracle's on the same weights
    orc = OracleModel(eng)
    eng.capture(1)
    pos, tok = 100, 17
    eng.reset(pos, tok)
    for step in range(2):
        got_tok = int(eng.generate(1)[0])
        got = eng.logits(1)[0]
        am, want = orc.step(tok, pos)
        assert close(got[:syn.d["V"]], want[:syn.d["V"]]), step
        assert got_tok < syn.d["V"] and argmax_ok(got_tok, want)
        tok, pos = got_tok, pos + 1
    eng.close()


@pytest.mark.parametrize("tie", [False, True])
def test_bf16_head_quantised_at_load(tmp_path, tie):
    syn = Synth(str(tmp_path / "h"), layers=1, V=2048, head="bf16", tie=tie)
    eng = load(syn)
    H, V = eng.desc.hidden, 2048
    q = eng.to_host(mi.T_LM_Q, 0, np.uint32).reshape(H // 8, V)
    s = O.f16_bits_to_f32(eng.to_host(mi.T_LM_S, 0, np.uint16).reshape(H // 64, V)).astype(np.float64)
    k = np.arange(H)
    nib = ((q[k // 8, :] >> (4 * (k % 8))[:, None]) & 0xF).astype(np.float64)  # [H][V]
    deq = (nib - 8.0) * s[k // 64, :]
    w = syn.lm_w.astype(np.float64).T  # [H][V]
    amax = np.abs(w).reshape(H // 64, 64, V).max(axis=1)
    want_s = O.f16_bits_to_f32(O.f32_to_f16_bits((2 * amax / 15).astype(np.float32))).astype(np.float64)
    assert np.array_equal(s, want_s)
    # round to nearest within the clamp range [-8, 7] s: |w - deq| <= s / 2, plus 7.5 times the
    # f16 rounding of s at a group's positive extreme (amax = 7.5 s exactly before rounding)
    err = np.abs(w - deq)
    assert np.all(err <= 0.5 * s[k // 64, :] * (1 + 2 * 7.5 * 2.0 ** -11) + 1e-12)
    eng.close()


@pytest.mark.parametrize("tie", [False, True])
def test_int8_head_made_at_load(tmp_path, tie):
    """An engine built with the int8 lm_head: the checkpoint's 16-bit head (or the tied
    embeddings) quantised at load is bitwise the oracle's row quantiser (itself pinned against
    the reference's lm_head_int8.cc), and a decode step of the loaded model matches the oracle's
    step with the int8 head. A packed (int4) head is refused."""
    from test_gemv_i8w_gpu import untile
    syn = Synth(str(tmp_path / "i8"), layers=1, V=2048, head="bf16", tie=tie)
    path = syn.write(split=2)
    desc = mi.checkpoint_desc(path, max_len=512, max_rows=4)
    desc.lm_head_int8 = 1
    eng = mi.Engine(desc, seed=5)
    print(f"engine_load {path} (int8 head): {eng.load(path)}", flush=True)
    H, V = eng.desc.hidden, 2048
    q = untile(eng.to_host(mi.T_LM_I8, 0, np.int8), H, V)
    s = eng.to_host(mi.T_LM_I8_S, 0, np.float32)
    w = np.ascontiguousarray(syn.lm_w.astype(np.float32))  # [V][H]
    for n in range(0, V, 7):
        qr = np.zeros(H, np.int8)
        sr = O.lib().orc_quantise_row_int8(O._p(np.ascontiguousarray(w[n])), H, O._p(qr))
        assert np.float32(sr).view(np.uint32) == s[n].view(np.uint32) and np.array_equal(q[n], qr), n
    orc = OracleModel(eng)
    eng.capture(1)
    pos, tok = 60, 9
    eng.reset(pos, tok)
    for step in range(2):
        got_tok = int(eng.generate(1)[0])
        got = eng.logits(1)[0]
        am, want = orc.step(tok, pos)
        assert close(got, want), step
        assert argmax_ok(got_tok, want)
        tok, pos = got_tok, pos + 1
    eng.close()
    packed = Synth(str(tmp_path / "p8"), layers=1, V=2048)
    ppath = packed.write(split=1)
    d2 = mi.checkpoint_desc(ppath, max_len=512, max_rows=4)
    d2.lm_head_int8 = 1
    e2 = mi.Engine(d2, seed=5)
    with pytest.raises(mi.MiError, match="packed"):
        e2.load(ppath)
    e2.close()


def test_moe_tensors(tmp_path):
    syn = Synth(str(tmp_path / "m"), layers=1, H=512, experts=16, top_k=4, moe_inter=128, V=2048)
    eng = load(syn)
    H, E, MI = 512, 16, 128
    L = syn.layers[0]
    rn = (E + 1 + 15) // 16 * 16
    rows = np.zeros((rn, H), np.float32)
    rows[:E + 1] = L["router"]
    rt = np.empty(rn * H, np.uint16)
    O.lib().orc_f16w_tile(O._p(O.f32_to_f16_bits(rows)), H, rn, O._p(rt))
    assert np.array_equal(eng.to_host(mi.T_ROUTER, 0, np.uint16), rt)
    gu = eng.to_host(mi.T_MOE_GU, 0, np.uint32)
    dn = eng.to_host(mi.T_MOE_DN, 0, np.uint32)
    gub = (2 * MI // 16) * (H // 64) * 136
    dnb = (H // 16) * (MI // 64) * 136
    for e in (0, 7, E):  # two routed experts and the shared one (block E)
        (gq, gs), (uq, us), (dq, ds) = L["experts"][e]
        iq = np.ascontiguousarray(expect_interleave(gq, uq))
        is_ = np.ascontiguousarray(expect_interleave(gs, us))
        want = np.empty(gub, np.uint32)
        O.lib().orc_repack_layout1(O._p(iq), O._p(is_), H, 2 * MI, O._p(want))
        assert np.array_equal(gu[e * gub:(e + 1) * gub], want), e
        want = np.empty(dnb, np.uint32)
        O.lib().orc_repack_layout1(O._p(np.ascontiguousarray(dq)), O._p(np.ascontiguousarray(ds)), MI, H, O._p(want))
        assert np.array_equal(dn[e * dnb:(e + 1) * dnb], want), e
    eng.close()


def test_mismatched_engine_is_refused(tmp_path):
    syn = Synth(str(tmp_path / "x"), layers=1, V=2048)
    path = syn.write()
    desc = mi.checkpoint_desc(path, max_len=256)
    desc.inter = 2048  # not the checkpoint's
    eng = mi.Engine(desc, seed=1)
    with pytest.raises(mi.MiError) as e:
        eng.load(path)
    assert "does not match config.json" in str(e.value)
    eng.close()


def test_mtp_head_loaded_and_drafts(tmp_path):
    """An engine built with the MTP head loads the checkpoint's bf16 mtp.* tensors: every linear
    quantised at load bitwise as the oracle's restatement of rtn.h (itself pinned against the
    reference's rtn_int4_g64), in the main layers' layouts; the norms as shipped. The loaded
    head's three draft lists follow the oracle's head on the same weights."""
    from test_mtp_gpu import OracleHead, head_kv
    syn = Synth(str(tmp_path / "mtp"), layers=2, V=2048, mtp=True)
    path = syn.write(split=2)
    desc = mi.checkpoint_desc(path, max_len=512, max_rows=4)
    desc.mtp = 1
    eng = mi.Engine(desc, seed=5)
    rep = eng.load(path)
    print(f"engine_load {path} (MTP head): {rep}", flush=True)
    assert "MTP head: 15 tensors, 8 linears quantised" in rep
    d = eng.desc
    H, I, QH, KVH, HD, li = d.hidden, d.inter, d.q_heads, d.kv_heads, d.head_dim, d.layers

    def rtn(b, K, N):
        q = np.zeros((K // 8, N), np.uint32)
        s = np.zeros((K // 64, N), np.uint16)
        O.lib().orc_rtn_int4_g64(O._p(np.ascontiguousarray(b)), K, N, O._p(q), O._p(s))
        return q, s

    m = syn.mtp
    fq, fs = rtn(m["fc"], 2 * H, H)
    assert np.array_equal(eng.to_host(mi.T_MTP_FC_Q, 0, np.uint32), fq.ravel())
    assert np.array_equal(eng.to_host(mi.T_MTP_FC_S, 0, np.uint16), fs.ravel())
    q, k, v = rtn(m["q"], H, QH * HD), rtn(m["k"], H, KVH * HD), rtn(m["v"], H, KVH * HD)
    assert np.array_equal(eng.to_host(mi.T_QKV_Q, li, np.uint32), np.concatenate([q[0], k[0], v[0]], 1).ravel())
    assert np.array_equal(eng.to_host(mi.T_QKV_S, li, np.uint16), np.concatenate([q[1], k[1], v[1]], 1).ravel())
    o = rtn(m["o"], QH * HD, H)
    assert np.array_equal(eng.to_host(mi.T_O_Q, li, np.uint32), o[0].ravel())
    g, u, dn = rtn(m["gate"], H, I), rtn(m["up"], H, I), rtn(m["down"], I, H)
    assert np.array_equal(eng.to_host(mi.T_GU_Q, li, np.uint32), expect_interleave(g[0], u[0]).ravel())
    assert np.array_equal(eng.to_host(mi.T_GU_S, li, np.uint16), expect_interleave(g[1], u[1]).ravel())
    assert np.array_equal(eng.to_host(mi.T_DOWN_Q, li, np.uint32), dn[0].ravel())
    assert np.array_equal(eng.to_host(mi.T_DOWN_S, li, np.uint16), dn[1].ravel())
    for kind, layer, key in ((mi.T_MTP_PRE_E, 0, "pre_e"), (mi.T_MTP_PRE_H, 0, "pre_h"), (mi.T_MTP_FINAL, 0, "final"),
                             (mi.T_IN_NORM, li, "in_norm"), (mi.T_POST_NORM, li, "post_norm"),
                             (mi.T_Q_NORM, li, "q_norm"), (mi.T_K_NORM, li, "k_norm")):
        assert np.array_equal(eng.to_host(kind, layer, np.float32), m[key].astype(np.float32)), key
    # the loaded head drafts as the oracle's head on the same weights
    orc = OracleModel(eng)
    oh = OracleHead(eng, orc)
    eng.capture(1)
    eng.reset(100, 7)
    eng.generate(3)
    c = eng.ctrl()
    pos, cur = int(c[mi.CTRL_POS]), int(c[mi.CTRL_CUR])
    hh0 = eng.to_host(mi.T_MTP_HH, 0, np.uint16)[:H].copy()
    kk, vv = head_kv(eng)
    drafts = eng.draft(3)
    tok, h = cur, hh0
    for i in range(3):
        am, logits, hout = oh.run(tok, h, pos - 1 + i, kk, vv)
        assert argmax_ok(int(drafts[i]), logits), (i, drafts[i], am)
        tok, h = int(drafts[i]), hout
    eng.close()
    # an engine with the head refuses a checkpoint without one
    plain = Synth(str(tmp_path / "nomtp"), layers=1, V=2048)
    ppath = plain.write(split=1)
    d2 = mi.checkpoint_desc(ppath, max_len=512, max_rows=4)
    d2.mtp = 1
    e2 = mi.Engine(d2, seed=5)
    with pytest.raises(mi.MiError, match="no mtp.fc"):
        e2.load(ppath)
    e2.close()


def test_mtp_head_16bit_loaded_and_drafts(tmp_path):
    """desc.mtp_w16: the checkpoint's bf16 head linears kept in 16 bits as the reference's loader
    keeps a dense head (loader.cc:586-597), each the f16 of the bf16 weight in gemv_f16w's tiles
    (q||k||v and gate||up by output rows, gate / up interleaved in 16-row blocks), bitwise; the
    loaded head's drafts follow the oracle's 16-bit head on the same weights."""
    from test_mtp_gpu import OracleHead, head_kv
    syn = Synth(str(tmp_path / "mtp16"), layers=2, V=2048, mtp=True)
    path = syn.write(split=2)
    desc = mi.checkpoint_desc(path, max_len=512, max_rows=4)
    desc.mtp, desc.mtp_w16 = 1, 1
    eng = mi.Engine(desc, seed=5)
    rep = eng.load(path)
    print(f"engine_load {path} (16-bit MTP head): {rep}", flush=True)
    assert "MTP head: 15 tensors, 0 linears quantised" in rep and "kept 16-bit" in rep
    d = eng.desc
    H, I, QH, KVH, HD = d.hidden, d.inter, d.q_heads, d.kv_heads, d.head_dim

    def tiled(w_bf16_rows):
        w = O.f32_to_f16_bits(O.bf16_bits_to_f32(np.ascontiguousarray(w_bf16_rows)))
        N, K = w.shape
        t = np.zeros_like(w)
        O.lib().orc_f16w_tile(O._p(w), K, N, O._p(t))
        return t.ravel()

    m = syn.mtp
    n = np.arange(2 * I)
    gu_rows = np.where(n % 32 < 16, 0, I) + (n // 32) * 16 + n % 16
    want = {mi.T_MTP_W16_FC: m["fc"], mi.T_MTP_W16_QKV: np.concatenate([m["q"], m["k"], m["v"]]),
            mi.T_MTP_W16_O: m["o"], mi.T_MTP_W16_GU: np.concatenate([m["gate"], m["up"]])[gu_rows],
            mi.T_MTP_W16_DN: m["down"]}
    for kind, w in want.items():
        assert np.array_equal(eng.to_host(kind, 0, np.uint16), tiled(w)), kind
    orc = OracleModel(eng)
    oh = OracleHead(eng, orc)
    eng.capture(1)
    eng.reset(100, 7)
    eng.generate(3)
    c = eng.ctrl()
    pos, cur = int(c[mi.CTRL_POS]), int(c[mi.CTRL_CUR])
    hh0 = eng.to_host(mi.T_MTP_HH, 0, np.uint16)[:H].copy()
    kk, vv = head_kv(eng)
    drafts = eng.draft(3)
    tok, h = cur, hh0
    for i in range(3):
        am, logits, hout = oh.run(tok, h, pos - 1 + i, kk, vv)
        assert argmax_ok(int(drafts[i]), logits), (i, drafts[i], am)
        tok, h = int(drafts[i]), hout
    eng.close()


def test_moe_mtp_head_loaded_and_drafts(tmp_path):
    """An MoE model's head (spec 15e: one MoE layer of the model's shape) from bf16 mtp.*
    tensors: the router as f16 tiles, every expert's linears quantised by rtn.h's rule into
    layout-1 blocks, bitwise; the loaded head's drafts follow the oracle's head."""
    from test_mtp_gpu import OracleHead, head_kv
    H, E, MI = 512, 16, 128
    syn = Synth(str(tmp_path / "mm"), layers=1, H=H, experts=E, top_k=4, moe_inter=MI, V=2048, mtp=True)
    path = syn.write(split=2)
    desc = mi.checkpoint_desc(path, max_len=512, max_rows=4)
    desc.mtp = 1
    eng = mi.Engine(desc, seed=5)
    rep = eng.load(path)
    print(f"engine_load {path} (MoE MTP head): {rep}", flush=True)
    nq = 5 + 3 * (E + 1)  # fc, q, k, v, o and the experts' linears
    assert f"MTP head: {12 + 2 + 3 * (E + 1)} tensors, {nq} linears quantised" in rep
    li = eng.desc.layers
    m = syn.mtp
    rn = (E + 1 + 15) // 16 * 16
    rows = np.zeros((rn, H), np.float32)
    rows[:E + 1] = m["router"]
    rt = np.empty(rn * H, np.uint16)
    O.lib().orc_f16w_tile(O._p(O.f32_to_f16_bits(rows)), H, rn, O._p(rt))
    assert np.array_equal(eng.to_host(mi.T_ROUTER, li, np.uint16), rt)
    gu = eng.to_host(mi.T_MOE_GU, li, np.uint32)
    dn = eng.to_host(mi.T_MOE_DN, li, np.uint32)
    gub, dnb = (2 * MI // 16) * (H // 64) * 136, (H // 16) * (MI // 64) * 136

    def rtn(b, K, N):
        q = np.zeros((K // 8, N), np.uint32)
        s = np.zeros((K // 64, N), np.uint16)
        O.lib().orc_rtn_int4_g64(O._p(np.ascontiguousarray(b)), K, N, O._p(q), O._p(s))
        return q, s

    for e in (0, 9, E):
        (gq, gs), (uq, us), (dq, ds) = rtn(m["experts"][e][0], H, MI), rtn(m["experts"][e][1], H, MI), \
            rtn(m["experts"][e][2], MI, H)
        want = np.empty(gub, np.uint32)
        O.lib().orc_repack_layout1(O._p(np.ascontiguousarray(expect_interleave(gq, uq))),
                                   O._p(np.ascontiguousarray(expect_interleave(gs, us))), H, 2 * MI, O._p(want))
        assert np.array_equal(gu[e * gub:(e + 1) * gub], want), e
        want = np.empty(dnb, np.uint32)
        O.lib().orc_repack_layout1(O._p(dq), O._p(ds), MI, H, O._p(want))
        assert np.array_equal(dn[e * dnb:(e + 1) * dnb], want), e
    orc = OracleModel(eng)
    oh = OracleHead(eng, orc)
    eng.capture(1)
    eng.reset(100, 7)
    eng.generate(3)
    c = eng.ctrl()
    pos, cur = int(c[mi.CTRL_POS]), int(c[mi.CTRL_CUR])
    hh0 = eng.to_host(mi.T_MTP_HH, 0, np.uint16)[:H].copy()
    kk, vv = head_kv(eng)
    drafts = eng.draft(3)
    tok, h = cur, hh0
    for i in range(3):
        am, logits, hout = oh.run(tok, h, pos - 1 + i, kk, vv)
        assert argmax_ok(int(drafts[i]), logits), (i, drafts[i], am)
        tok, h = int(drafts[i]), hout
    eng.close()

"""The GEMV's fused epilogues (one consumer work-group per 64-column tile) and the fused
embed + first norm, against the separate-kernel chain they replace, bit for bit on the
same partials: prep_res_fold at 64-element chunks + prep_norm_finish, prep_silu_mul,
the lm_head fold + argmax (tests/kernels/prep_test.cc, argmax_test.cc's bars). Every
launch must leave its hand-off words empty again, so a replay gives the same bits.
Each test runs twice: with the fixed consumers (slice S-1, QKV's extra row) and with an
arrival array (the last slice to arrive consumes), which must give the same bits and leave
the array at zero."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16
L = O.lib


def rand_w(K, N, seed):
    rng = np.random.default_rng(seed)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_f16_bits(rng.uniform(0.002, 0.02, size=(K // 64, N)).astype(np.float32))
    return qw, sc


EMPTY = 0xFFFFFFFF


def handoff(n):
    """n hand-off words set empty by the library's own initialiser"""
    d = empty((n,), np.float32)
    mi.call("mi_gemv_handoff_init", ptr(d), n, stream())
    return d


def all_empty(d, n=None):
    h = host(d, np.uint32).ravel()
    return bool(np.all(h[:n] == EMPTY))


MODE = {"consumers": "fixed"}


@pytest.fixture(autouse=True, params=["fixed", "arrive"])
def consumers(request):
    MODE["consumers"] = request.param
    yield request.param
    MODE["consumers"] = "fixed"


def launch_ex(dq, ds, dx, dpart, M, K, N, S, ep):
    """mi_gemv_w4a16_ex with this test's consumer mode; the arrival words must end at zero"""
    arr = None
    if MODE["consumers"] == "arrive":
        arr = dev(np.zeros(32 * (N // 64 + 1), np.uint32))
        ep.arrive = ptr(arr)
    mi.call("mi_gemv_w4a16_ex", ptr(dq), ptr(ds), ptr(dx), ptr(dpart), M, K, N, S, C.byref(ep), stream())
    if arr is not None:
        sync()
        assert not host(arr, np.uint32).any(), "arrival words not back at zero"


def partials_of(dq, ds, dx, M, K, N, S):
    part = empty((S, M, N), np.float32)
    mi.call("mi_gemv_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(part), M, K, N, S, stream())
    sync()
    return host(part, np.float32).copy()


@pytest.mark.parametrize("M,S,K,N", [(1, 8, 2048, 1024), (3, 4, 2048, 1024), (16, 1, 2048, 1024),
                                     (16, 8, 2048, 1024), (1, 34, 17408 // 8, 1024), (16, 2, 1024, 16384)])
def test_resid_epilogue_bitwise(M, S, K, N):
    # N = hidden; (1, 34): down's split width over 34 k-groups; (16, 2, N 16384): the
    # consumers' sums of squares polled in two rounds of rows
    qw, sc = rand_w(K, N, 10 + M)
    rng = np.random.default_rng(M)
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    resid = O.f32_to_f16_bits(rng.standard_normal((M, N)).astype(np.float32))
    w = (1 + 0.02 * rng.standard_normal(N)).astype(np.float32)
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    part = partials_of(dq, ds, dx, M, K, N, S)
    print(f"resid epilogue M={M} S={S} K={K} N={N}", flush=True)
    G = N // 64
    dr, dw = dev(resid), dev(w)
    dss = handoff(G * M * G)
    drs = empty((M,), np.float32)
    dxn = empty((M, N), np.uint16)
    dpart = handoff(S * M * N)
    ep = mi.GemvEpilogue(mi.EPI_RESID, ptr(dr), ptr(dss), ptr(drs), ptr(dw), ptr(dxn), 1e-6,
                         None, None, None, 0)
    r_ref = resid.copy()
    s_ref = np.zeros((G, M), np.float32)
    x_ref = np.zeros((M, N), np.uint16)
    L().orc_res_fold(F16, O._p(part), O._p(r_ref), O._p(s_ref), M, N, S, G)
    L().orc_norm_finish(F16, O._p(s_ref), O._p(r_ref), O._p(w), O._p(x_ref), M, N, G, 1e-6)
    rstd_ref = np.zeros(M, np.float32)
    for m in range(M):
        tot = np.float32(0)
        for g in range(G):
            tot = np.float32(tot + s_ref[g, m])
        rstd_ref[m] = np.float32(1) / np.sqrt(np.float32(tot / np.float32(N) + np.float32(1e-6)))
    for rep in range(2):  # a replay must find the hand-off words empty again
        if rep:
            dr.copy_(dev(resid))
        launch_ex(dq, ds, dx, dpart, M, K, N, S, ep)
        sync()
        assert all_empty(dpart) and all_empty(dss)
        assert np.array_equal(host(dr, np.uint16), r_ref)
        assert np.array_equal(host(dxn, np.uint16), x_ref)
        assert np.array_equal(host(drs, np.uint32), rstd_ref.view(np.uint32))


@pytest.mark.parametrize("M,S", [(1, 4), (4, 2)])
def test_silu_epilogue(M, S):
    K, I = 1024, 1536
    N = 2 * I
    qw, sc = rand_w(K, N, 20 + M)
    x = O.f32_to_f16_bits(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    part = partials_of(dq, ds, dx, M, K, N, S)
    dh = empty((M, I), np.uint16)
    dpart = handoff(S * M * N)
    ep = mi.GemvEpilogue(mi.EPI_SILU, None, None, None, None, None, 0.0, ptr(dh), None, None, 0)
    launch_ex(dq, ds, dx, dpart, M, K, N, S, ep)
    sync()
    assert all_empty(dpart)
    got = host(dh, np.uint16)
    want = O.silu_mul(F16, part, M, I, S)
    a = O.f16_bits_to_f32(got).astype(np.float64)
    b = O.f16_bits_to_f32(want).astype(np.float64)
    assert np.all(np.abs(a - b) <= 2 * np.maximum(np.abs(b), 2.0 ** -14) * 2.0 ** -10)
    assert np.mean(got == want) >= 0.95


@pytest.mark.parametrize("M", [1, 3])
def test_logits_epilogue_and_argmax(M):
    K, V, used = 1024, 8192, 8000
    qw, sc = rand_w(K, V, 30 + M)
    x = O.f32_to_f16_bits(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    S = 4
    part = partials_of(dq, ds, dx, M, K, V, S)
    dl = empty((M, V), np.float32)
    dap = empty((M * (V // 64) * 2,), np.uint32)
    dpart = handoff(S * M * V)
    ep = mi.GemvEpilogue(mi.EPI_LOGITS, None, None, None, None, None, 0.0, None, ptr(dl), ptr(dap), used)
    launch_ex(dq, ds, dx, dpart, M, K, V, S, ep)
    c = np.zeros(64, np.uint32)
    c[1] = M
    ctrl = dev(c)
    mi.call("mi_argmax_finish", ptr(ctrl), ptr(dap), V // 64, None, 0, stream())
    sync()
    assert all_empty(dpart)
    want = np.zeros((M, V), np.float32)
    for s in range(S):
        want = want + part[s]  # ascending s from 0.f
    got = host(dl, np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    cc = host(ctrl, np.uint32)
    assert list(cc[10:10 + M]) == [O.argmax(want[m], used) for m in range(M)]


@pytest.mark.parametrize("M,S", [(1, 8), (3, 4)])
def test_f16out_epilogue_is_gemv_then_fold(M, S):
    """MI_EPI_F16OUT: the fold of the S partials to fp16 inside the GEMV launch, bitwise
    mi_gemv_w4a16 followed by mi_fold_partials (the oracle's fold: ascending s from +0)."""
    K = N = 4096
    qw, sc = rand_w(K, N, 50 + M)
    x = O.f32_to_f16_bits(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    part = partials_of(dq, ds, dx, M, K, N, S)
    want = np.zeros((M, N), np.float32)
    for s in range(S):
        want = want + part[s]
    out = empty((M, N), np.uint16)
    dpart = handoff(S * M * N)
    ep = mi.GemvEpilogue(kind=mi.EPI_F16OUT, out16=ptr(out))
    for _ in range(2):  # the hand-off words are empty again: a second launch gives the same bits
        launch_ex(dq, ds, dx, dpart, M, K, N, S, ep)
        sync()
        assert all_empty(dpart)
        assert np.array_equal(host(out, np.uint16), O.f32_to_f16_bits(want))


def test_launches_share_handoff_words():
    """The engine's pattern: fused launches of different shapes and split widths take turns
    on one hand-off buffer; each finds it empty and leaves it so."""
    K, N = 1024, 2048
    rng = np.random.default_rng(77)
    shapes = [(K, N, 8), (K, 2 * N, 4), (2 * K, N, 16), (K, N, 1), (K, N, 8)]
    dpart = handoff(16 * 2 * N)
    for i, (k, n, S) in enumerate(shapes):
        qw, sc = rand_w(k, n, 90 + i)
        x = O.f32_to_f16_bits(rng.standard_normal((1, k)).astype(np.float32))
        dq, ds, dx = dev(qw), dev(sc), dev(x)
        part = partials_of(dq, ds, dx, 1, k, n, S)
        want = np.zeros((1, n), np.float32)
        for s_ in range(S):
            want = want + part[s_]
        out = empty((1, n), np.uint16)
        ep = mi.GemvEpilogue(kind=mi.EPI_F16OUT, out16=ptr(out))
        launch_ex(dq, ds, dx, dpart, 1, k, n, S, ep)
        sync()
        assert all_empty(dpart), i
        assert np.array_equal(host(out, np.uint16), O.f32_to_f16_bits(want)), i


@pytest.mark.parametrize("QH,KVH,HD,rot,M,n_act,paged,qk_norm,S", [
    (40, 8, 128, 128, 1, 1, False, True, 20), (40, 8, 128, 128, 3, 2, True, True, 8),
    (16, 2, 256, 64, 1, 1, False, False, 4), (16, 2, 256, 256, 4, 4, True, True, 2)])
def test_qkv_epilogue_is_gemv_then_attn_prep(QH, KVH, HD, rot, M, n_act, paged, qk_norm, S):
    """MI_EPI_QKV: attn_prep on the folded q||k||v inside the GEMV launch, bitwise the plain
    GEMV followed by mi_attn_prep (attn_q, the K/V cache rows written, nothing else touched)."""
    sh = O.attn_shape(QH, KVH, HD, rot_dim=rot)
    msh = mi.lib_shape(sh)
    K, N = 64 * S * max(1, 16 // S), sh.qkv_n
    pos, Lm, P = 517, 1024, 64
    rng = np.random.default_rng(QH + M)
    qw, sc = rand_w(K, N, 60 + M)
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    qn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk_norm else None
    kn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk_norm else None
    rope = O.rope_table(1e6, rot, Lm)
    pages = rng.permutation(Lm // P).astype(np.uint32) if paged else None
    kk = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    vv = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    keep = [dev(qn) if qk_norm else None, dev(kn) if qk_norm else None, dev(rope), dev(pages) if paged else None]
    pnorm = [ptr(k) if k is not None else None for k in keep]
    print(f"qkv epilogue {QH}/{KVH}x{HD} rot {rot} M={M} n_act={n_act} paged={paged} S={S}", flush=True)

    def ctrl():
        c = np.zeros(64, np.uint32)
        c[0], c[1] = pos, n_act
        return dev(c)

    # the plain GEMV, then attn_prep
    part = empty((S, M, N), np.float32)
    mi.call("mi_gemv_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(part), M, K, N, S, stream())
    c1, aq1, k1, v1 = ctrl(), empty((M, QH, HD), np.float32), dev(kk), dev(vv)
    aq1.zero_()
    mi.call("mi_attn_prep", ptr(c1), ptr(part), S, M, mi.shape_ref(sh), pnorm[0], pnorm[1], pnorm[2], ptr(aq1), None,
            ptr(k1), ptr(v1), HD, Lm * HD, pnorm[3], P if paged else 0, Lm, stream())
    # the fused launch, twice (the hand-off words are empty again after the first)
    dpart = handoff(S * M * N)
    for rep in range(2):
        c2, aq2, k2, v2 = ctrl(), empty((M, QH, HD), np.float32), dev(kk), dev(vv)
        aq2.zero_()
        ep = mi.GemvEpilogue(kind=mi.EPI_QKV, ctrl=ptr(c2), shape=C.cast(C.pointer(msh), C.c_void_p),
                             q_norm=pnorm[0], k_norm=pnorm[1], rope=pnorm[2], attn_q=ptr(aq2), kv_k=ptr(k2),
                             kv_v=ptr(v2), row_stride=HD, head_stride=Lm * HD, pages=pnorm[3],
                             page=P if paged else 0, kv_len=Lm)
        launch_ex(dq, ds, dx, dpart, M, K, N, S, ep)
        sync()
        assert all_empty(dpart)
        assert np.array_equal(host(aq2, np.uint32), host(aq1, np.uint32)), rep
        assert np.array_equal(host(k2, np.uint16), host(k1, np.uint16)), rep
        assert np.array_equal(host(v2, np.uint16), host(v1, np.uint16)), rep
        assert np.array_equal(host(c2, np.uint32), host(c1, np.uint32)), rep


def test_qkv_epilogue_past_the_cache():
    """A position at or past kv_len writes nothing and flags the step (attn_prep's rule)."""
    sh = O.attn_shape(40, 8, 128)
    msh = mi.lib_shape(sh)
    K, N, S, Lm = 1024, sh.qkv_n, 4, 256
    qw, sc = rand_w(K, N, 7)
    x = O.f32_to_f16_bits(np.random.default_rng(7).standard_normal((1, K)).astype(np.float32))
    rope = dev(O.rope_table(1e6, 128, Lm + 8))
    c = np.zeros(64, np.uint32)
    c[0], c[1] = Lm, 1
    dc = dev(c)
    kk = np.full((8, Lm, 128), 7, np.uint16)
    k2, v2 = dev(kk), dev(kk)
    aq = dev(np.zeros((1, 40, 128), np.float32))
    dpart = handoff(S * N)
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    ep = mi.GemvEpilogue(kind=mi.EPI_QKV, ctrl=ptr(dc), shape=C.cast(C.pointer(msh), C.c_void_p), rope=ptr(rope),
                         attn_q=ptr(aq), kv_k=ptr(k2), kv_v=ptr(v2), row_stride=128, head_stride=Lm * 128,
                         kv_len=Lm)
    launch_ex(dq, ds, dx, dpart, 1, K, N, S, ep)
    sync()
    assert all_empty(dpart)
    assert host(dc, np.uint32)[18] == 0xDEAD0002
    assert np.array_equal(host(k2, np.uint16), kk) and np.array_equal(host(v2, np.uint16), kk)
    assert not host(aq, np.uint32).any()


def test_embed_norm_bitwise():
    V, H, M = 512, 5120, 2
    rng = np.random.default_rng(4)
    emb = O.f32_to_f16_bits(rng.standard_normal((V, H)).astype(np.float32))
    w = (1 + 0.02 * rng.standard_normal(H)).astype(np.float32)
    c = np.zeros(64, np.uint32)
    c[1], c[2], c[3] = M, 17, 300
    ctrl, demb, dw = dev(c), dev(emb), dev(w)
    dr = empty((M, H), np.uint16)
    dx = empty((M, H), np.uint16)
    drs = empty((M,), np.float32)
    mi.call("mi_embed_norm", ptr(ctrl), ptr(demb), ptr(dr), ptr(dw), ptr(dx), ptr(drs), M, H, V, 1e-6, stream())
    sync()
    r_ref = emb[[17, 300]].copy()
    G = H // 64
    s_ref = np.zeros((G, M), np.float32)
    x_ref = np.zeros((M, H), np.uint16)
    L().orc_res_fold(F16, None, O._p(r_ref), O._p(s_ref), M, H, 0, G)
    L().orc_norm_finish(F16, O._p(s_ref), O._p(r_ref), O._p(w), O._p(x_ref), M, H, G, 1e-6)
    assert np.array_equal(host(dr, np.uint16), r_ref)
    assert np.array_equal(host(dx, np.uint16), x_ref)


@pytest.mark.parametrize("kind", ["resid", "silu"])
def test_handoff_timeout_sets_the_status_word(kind):
    """A consumer whose hand-off words never fill gives up after poll_limit polls, sets the
    status word and exits (fault injection from the host: the producers publish nothing, and
    the poll limit is tiny, so every kernel still ends normally). The words are left empty, and
    the next normal launch on the same words gives the normal result."""
    M, K, S = 1, 1024, 4
    N = 1024
    qw, sc = rand_w(K, N, 77)
    rng = np.random.default_rng(5)
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    part = partials_of(dq, ds, dx, M, K, N, S)
    dpart = handoff(S * M * N)
    status = dev(np.zeros(1, np.uint32))
    G = N // 64
    if kind == "resid":
        resid = O.f32_to_f16_bits(rng.standard_normal((M, N)).astype(np.float32))
        w = np.ones(N, np.float32)
        dr, dw = dev(resid), dev(w)
        dss = handoff(G * M * G)
        drs = empty((M,), np.float32)
        dout = empty((M, N), np.uint16)
        ep = mi.GemvEpilogue(kind=mi.EPI_RESID, resid=ptr(dr), sumsq=ptr(dss), rstd=ptr(drs), next_norm_w=ptr(dw),
                             x_next=ptr(dout), eps=1e-6)
    else:
        dout = empty((M, N // 2), np.uint16)
        ep = mi.GemvEpilogue(kind=mi.EPI_SILU, h=ptr(dout))
    ep.status, ep.poll_limit, ep.inject = ptr(status), 64, 1
    print(f"handoff timeout {kind}: injected launch", flush=True)
    launch_ex(dq, ds, dx, dpart, M, K, N, S, ep)
    sync()
    assert int(host(status, np.uint32)[0]) == mi.STATUS_HANDOFF_TIMEOUT
    assert all_empty(dpart)
    if kind == "resid":
        assert all_empty(dss)
    # a normal launch afterwards: status untouched, result as the oracle's
    status.zero_()
    ep.poll_limit, ep.inject = 0, 0
    if kind == "resid":
        dr.copy_(dev(resid))
    print(f"handoff timeout {kind}: normal launch", flush=True)
    launch_ex(dq, ds, dx, dpart, M, K, N, S, ep)
    sync()
    assert int(host(status, np.uint32)[0]) == 0
    if kind == "resid":
        r_ref = resid.copy()
        s_ref = np.zeros((G, M), np.float32)
        x_ref = np.zeros((M, N), np.uint16)
        L().orc_res_fold(F16, O._p(part), O._p(r_ref), O._p(s_ref), M, N, S, G)
        L().orc_norm_finish(F16, O._p(s_ref), O._p(r_ref), O._p(w), O._p(x_ref), M, N, G, 1e-6)
        assert np.array_equal(host(dout, np.uint16), x_ref)
    else:
        want = O.silu_mul(F16, part, M, N // 2, S)
        a = O.f16_bits_to_f32(host(dout, np.uint16)).astype(np.float64)
        b = O.f16_bits_to_f32(want).astype(np.float64)
        assert np.all(np.abs(a - b) <= 2 * np.maximum(np.abs(b), 2.0 ** -14) * 2.0 ** -10)

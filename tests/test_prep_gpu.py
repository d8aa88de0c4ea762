"""Between-GEMV kernels and the token boundary on the GPU vs the CPU oracle (fp16).

Bars (tests/kernels/prep_test.cc, embed_gather_test.cc, argmax_test.cc): residual fold and
RMSNorm bit-exact (same per-element chain, same 256-lane tree); silu within 2 fp16 ulp
(exp), exact at the exp-free point; q/k-norm + RoPE + KV write bit-exact; embed_gather a
verbatim copy with the bad-id flag; argmax indices exact with ties to the lower index and
the masked tail, and the control block advanced exactly."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16
L = O.lib


def ctrl_dev(pos=0, n_act=1, cur=(0,)):
    c = np.zeros(64, np.uint32)
    c[0], c[1] = pos, n_act
    c[2:2 + len(cur)] = cur
    return dev(c)


def ulp16_diff(a, b):
    a = O.f16_bits_to_f32(a).astype(np.float64)
    b = O.f16_bits_to_f32(b).astype(np.float64)
    u = np.maximum(np.abs(b), 2.0 ** -14) * 2.0 ** -10
    return np.abs(a - b) / u


@pytest.mark.parametrize("S_PREV,M", [(0, 1), (1, 1), (4, 3), (17, 1)])
def test_res_fold_norm_finish_bitwise(S_PREV, M):
    K, G = 5120, 20
    rng = np.random.default_rng(S_PREV * 10 + M)
    part = (rng.standard_normal((max(S_PREV, 1), M, K)) * 0.5).astype(np.float32)
    resid = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = (1 + 0.02 * rng.standard_normal(K)).astype(np.float32)
    print(f"res_fold S_PREV={S_PREV} M={M}", flush=True)
    dp, dr, dw = dev(part), dev(resid), dev(w)
    ss = empty((G, M), np.float32)
    dx = empty((M, K), np.uint16)
    mi.call("mi_res_fold", ptr(dp), ptr(dr), ptr(ss), M, K, S_PREV, G, stream())
    mi.call("mi_norm_finish", ptr(ss), ptr(dr), ptr(dw), ptr(dx), M, K, G, 1e-6, stream())
    sync()
    r_ref = resid.copy()
    s_ref = np.zeros((G, M), np.float32)
    x_ref = np.zeros((M, K), np.uint16)
    L().orc_res_fold(F16, O._p(part), O._p(r_ref), O._p(s_ref), M, K, S_PREV, G)
    L().orc_norm_finish(F16, O._p(s_ref), O._p(r_ref), O._p(w), O._p(x_ref), M, K, G, 1e-6)
    assert np.array_equal(host(dr, np.uint16), r_ref)
    assert np.array_equal(host(ss, np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(host(dx, np.uint16), x_ref)


@pytest.mark.parametrize("S_PREV,K", [(0, 5120), (4, 5120), (2, 2048)])
def test_res_norm_bitwise(S_PREV, K):
    M = 2
    rng = np.random.default_rng(K + S_PREV)
    part = (rng.standard_normal((max(S_PREV, 1), M, K)) * 0.5).astype(np.float32)
    resid = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    w = (1 + 0.02 * rng.standard_normal(K)).astype(np.float32)
    dp, dr, dw = dev(part), dev(resid), dev(w)
    dx = empty((M, K), np.uint16)
    mi.call("mi_res_norm", ptr(dp), ptr(dr), ptr(dw), ptr(dx), M, K, S_PREV, 1e-6, stream())
    sync()
    r_ref, x_ref = O.res_norm(F16, part, resid, w, M, K, S_PREV)
    assert np.array_equal(host(dr, np.uint16), r_ref)
    assert np.array_equal(host(dx, np.uint16), x_ref)


def test_silu_mul():
    M, N, S = 2, 17408, 8
    rng = np.random.default_rng(5)
    part = (rng.standard_normal((S, M, 2 * N)) * 1.5).astype(np.float32)
    gcol = lambda k: (k // 16) * 32 + k % 16
    part[:, 0, gcol(7)] = 0.0
    part[0, 0, gcol(7)] = 30.0  # silu(30) = 30 exactly in fp32: an exp-free point
    dp = dev(part)
    dx = empty((M, N), np.uint16)
    mi.call("mi_silu_mul", ptr(dp), ptr(dx), M, N, S, stream())
    sync()
    got = host(dx, np.uint16)
    want = O.silu_mul(F16, part, M, N, S)
    d = ulp16_diff(got, want)
    assert d.max() <= 2.0
    assert np.mean(got == want) >= 0.95
    assert got[0, 7] == want[0, 7]


def _prep_case(sh, M, n_act, pos, S, Lm, paged, qk_norm, seed):
    rng = np.random.default_rng(seed)
    HD, QH, KVH = sh.head_dim, sh.q_heads, sh.kv_heads
    part = rng.standard_normal((S, M, sh.qkv_n)).astype(np.float32)
    qn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk_norm else None
    kn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk_norm else None
    rope = O.rope_table(1e6, sh.rot_dim, Lm)
    P = 64
    pages = rng.permutation(Lm // P).astype(np.uint32) if paged else None
    kk = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    vv = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    return part, qn, kn, rope, pages, P, kk, vv


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("paged", [False, True])
def test_attn_prep_bitwise(gated, paged):
    if gated:
        sh = O.attn_shape(24, 4, 256, rot_dim=64, gated=True)
    else:
        sh = O.attn_shape(40, 8, 128)
    M, n_act, pos, S, Lm = 3, 2, 517, 2, 1024
    part, qn, kn, rope, pages, P, kk, vv = _prep_case(sh, M, n_act, pos, S, Lm, paged, True, 3)
    HD, QH, KVH = sh.head_dim, sh.q_heads, sh.kv_heads
    print(f"attn_prep gated={gated} paged={paged}", flush=True)
    ctrl = ctrl_dev(pos, n_act)
    dq = empty((M, QH, HD), np.float32)
    dg = empty((M, QH, HD), np.float32)
    dq.zero_(); dg.zero_()
    dk, dv = dev(kk), dev(vv)
    dpages = dev(pages) if paged else None
    shp = C.byref(sh)  # mi_attn_shape and orc_attn_shape share one layout
    keep = [dev(part), dev(qn), dev(kn), dev(rope)]  # held until the kernel has run
    mi.call("mi_attn_prep", ptr(ctrl), ptr(keep[0]), S, M, shp, ptr(keep[1]), ptr(keep[2]), ptr(keep[3]),
            ptr(dq), ptr(dg), ptr(dk), ptr(dv), HD, Lm * HD, ptr(dpages), P if paged else 0, Lm, stream())
    sync()
    aq = np.zeros((M, QH, HD), np.float32)
    ag = np.zeros((M, QH, HD), np.float32)
    k2, v2 = kk.copy(), vv.copy()
    L().orc_attn_prep(F16, shp, pos, n_act, M, O._p(part), S, O._p(qn), O._p(kn), O._p(rope), O._p(aq),
                      O._p(ag), O._p(k2), O._p(v2), HD, Lm * HD, O._p(pages), P if paged else 0)
    assert np.array_equal(host(dq, np.uint32)[:n_act], aq.view(np.uint32)[:n_act])
    if gated:
        assert np.array_equal(host(dg, np.uint32)[:n_act], ag.view(np.uint32)[:n_act])
    assert np.array_equal(host(dk, np.uint16), k2)
    assert np.array_equal(host(dv, np.uint16), v2)


def test_attn_prep_without_qk_norm():
    sh = O.attn_shape(16, 2, 256)
    M, n_act, pos, S, Lm = 1, 1, 40, 4, 128
    part, qn, kn, rope, pages, P, kk, vv = _prep_case(sh, M, n_act, pos, S, Lm, False, False, 9)
    HD, QH = sh.head_dim, sh.q_heads
    ctrl = ctrl_dev(pos, n_act)
    dq = empty((M, QH, HD), np.float32)
    dk, dv = dev(kk), dev(vv)
    keep = [dev(part), dev(rope)]
    mi.call("mi_attn_prep", ptr(ctrl), ptr(keep[0]), S, M, mi.shape_ref(sh), None, None, ptr(keep[1]),
            ptr(dq), None, ptr(dk), ptr(dv), HD, Lm * HD, None, 0, Lm, stream())
    sync()
    aq = np.zeros((M, QH, HD), np.float32)
    k2, v2 = kk.copy(), vv.copy()
    L().orc_attn_prep(F16, C.byref(sh), pos, n_act, M, O._p(part), S, None, None, O._p(rope), O._p(aq),
                      None, O._p(k2), O._p(v2), HD, Lm * HD, None, 0)
    assert np.array_equal(host(dq, np.uint32), aq.view(np.uint32))
    assert np.array_equal(host(dk, np.uint16), k2) and np.array_equal(host(dv, np.uint16), v2)


def test_embed_gather_and_bad_id():
    V, H = 1000, 5120
    emb = np.random.default_rng(1).integers(0, 0x7C00, (V, H)).astype(np.uint16)
    demb = dev(emb)
    ctrl = ctrl_dev(0, 2, (17, 999))
    out = dev(np.full((2, H), 7, np.uint16))
    mi.call("mi_embed_gather", ptr(ctrl), ptr(demb), ptr(out), 2, H, V, stream())
    sync()
    assert np.array_equal(host(out, np.uint16), emb[[17, 999]])
    assert host(ctrl, np.uint32)[18] == 0
    ctrl = ctrl_dev(0, 1, (V,))
    out = dev(np.full((1, H), 7, np.uint16))
    mi.call("mi_embed_gather", ptr(ctrl), ptr(demb), ptr(out), 1, H, V, stream())
    sync()
    assert np.all(host(out, np.uint16) == 7)
    assert host(ctrl, np.uint32)[18] == 0xDEAD0001


def test_argmax_cases_and_control_block():
    """tests/kernels/argmax_test.cc's cases at vocab 151936 (masked tail for one case),
    replayed on one control block: out_token, cur_token, pos advance, history."""
    V = 151936
    bg = lambda s: np.random.default_rng(s).uniform(-4, -1, V).astype(np.float32)
    cases = []
    v = bg(11); v[123456] = 3.5; cases.append((v, V, 123456))
    v = bg(12); v[5000] = v[5001] = v[90000] = 7.0; cases.append((v, V, 5000))
    v = bg(13); v[V - 100] = 99.0; v[V - 20] = 100.0; v[1000] = 42.0; cases.append((v, V - 100, 1000))
    cases.append((np.zeros(V, np.float32), V, 0))
    v = bg(14); v[V - 1] = 5.0; cases.append((v, V, V - 1))
    v = bg(15); cases.append((v, V, int(np.argmax(v))))
    ctrl = ctrl_dev(17, 1)
    groups = mi.lib().mi_argmax_groups(V)
    part = empty((groups * 2,), np.uint32)
    hist = dev(np.zeros(16, np.uint32))
    for i, (lg, used, want) in enumerate(cases):
        dl = dev(lg)
        mi.call("mi_argmax", ptr(ctrl), ptr(dl), ptr(part), ptr(hist), 16, 1, V, used, stream())
        sync()
        c = host(ctrl, np.uint32)
        assert c[10] == want and c[2] == want, (i, c[10], want)
        assert c[0] == 17 + i + 1 and c[19] == i + 1
        assert host(hist, np.uint32)[i] == want
        assert O.argmax(lg, used) == want


def test_argmax_rows():
    V, M = 4096, 3
    rng = np.random.default_rng(2)
    lg = rng.standard_normal((M, V)).astype(np.float32)
    lg[1, 100] = lg[1, 3000] = 50.0
    ctrl = ctrl_dev(5, M)
    part = empty((mi.lib().mi_argmax_groups(V) * M * 2,), np.uint32)
    dl = dev(lg)
    mi.call("mi_argmax", ptr(ctrl), ptr(dl), ptr(part), None, 0, M, V, V, stream())
    sync()
    c = host(ctrl, np.uint32)
    want = [O.argmax(lg[m]) for m in range(M)]
    assert list(c[10:13]) == want and want[1] == 100
    assert c[2] == want[-1] and c[0] == 5 + M

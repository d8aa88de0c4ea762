"""The chunked prefill on the GPU: the int4 linear for many rows on the matrix cores, the chunk's
causal attention, and Engine::prefill against decode's ingest of the same ids on one engine
(tests/prefill/prefill_consistency_test.cc's comparison: prefill against decode-ingest, same
engine, same prompt).

Bars: the GEMM within 2^-16 sum |x w| of the fp64 product of the same f16-rounded weights
(w = f16((q - 8) scale)), exact where every operation is exact; the attention within rel 2e-3 of
fp64 causal softmax attention, cosine >= 0.99999, paged bitwise the contiguous cache; the engine's
prefill leaves the control block as ingest does (pos, cur_token unless the last logits' top two are
closer than the tolerance), the KV rows and the last logits within the two paths' rounding
difference (prefill rounds each dequantised weight to f16; decode's GEMV multiplies the exact
integers and scales once per group)."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from mipkg import dev, empty, host, mi, ptr, stream, sync
from test_engine_gpu import OracleModel, close, small_desc

pytestmark = pytest.mark.gpu
F16 = O.ORC_F16


def weights(K, N, seed, exact=False):
    rng = np.random.default_rng(seed)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    if exact:
        sc = np.full((K // 64, N), O.f32_to_f16_bits(np.float32(1 / 16)), np.uint16)
    else:
        sc = O.f32_to_f16_bits(rng.uniform(0.002, 0.02, size=(K // 64, N)).astype(np.float32))
    return qw, sc


def dequant16(qw, sc):
    """w[k][n] = f16((q - 8) * s): the product of two f16 values is exact in fp32, so one
    rounding to f16 is the correctly rounded f16 product"""
    K = qw.shape[0] * 8
    k = np.arange(K)
    q = (qw[k // 8, :] >> (4 * (k % 8))[:, None]) & 0xF
    s = O.f16_bits_to_f32(sc)[k // 64, :]
    return ((q.astype(np.float32) - 8) * s).astype(np.float16).astype(np.float64)


# the shapes take all four work-group tiles on a 256-CU part (N % 256 != 0: 128 x 128; small
# grids: 64 x 256; T = 2000, N = 5120: 96 x 256; T = 1000, N = 14336: 128 x 256), with ragged T
# and odd group counts
@pytest.mark.parametrize("T,K,N", [(1, 256, 128), (3, 64, 256), (9, 320, 384), (37, 1024, 384), (130, 2048, 256),
                                   (256, 5120, 512), (1000, 192, 14336), (2000, 64, 5120)])
def test_gemm_vs_fp64(T, K, N):
    qw, sc = weights(K, N, T + K)
    x = O.f32_to_f16_bits(np.random.default_rng(T).standard_normal((T, K)).astype(np.float32))
    print(f"gemm T={T} K={K} N={N}", flush=True)
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    out = empty((T, N), np.float32)
    mi.call("mi_gemm_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(out), T, K, N, stream())
    sync()
    got = host(out, np.float32).astype(np.float64)
    w = dequant16(qw, sc)
    xf = O.f16_bits_to_f32(x).astype(np.float64)
    want = xf @ w
    bound = 2.0 ** -16 * (np.abs(xf) @ np.abs(w)) + 1e-30
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)


@pytest.mark.parametrize("T,K,N", [(70, 512, 256), (70, 512, 384), (1000, 128, 14336), (2000, 64, 5120)])
def test_gemm_exact_arithmetic(T, K, N):
    """Small-integer activations and scale 1/16: every product and partial sum is exact in fp32,
    so the GEMM equals the fp64 product bit for bit (any misplaced nibble, row or column shows)."""
    qw, sc = weights(K, N, 3, exact=True)
    x = O.f32_to_f16_bits(np.random.default_rng(4).integers(-3, 4, size=(T, K)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    out = empty((T, N), np.float32)
    mi.call("mi_gemm_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(out), T, K, N, stream())
    sync()
    want = O.f16_bits_to_f32(x).astype(np.float64) @ dequant16(qw, sc)
    assert np.array_equal(host(out, np.float32).astype(np.float64), want)


@pytest.mark.parametrize("T,K,I", [(77, 1024, 640), (70, 512, 576), (1000, 128, 7168), (2000, 64, 2560)])
def test_gemm_silu_is_gemm_then_silu_mul(T, K, I):
    """mi_gemm_w4a16_silu: SwiGLU in the GEMM's epilogue, bitwise mi_gemm_w4a16 followed by
    mi_silu_mul (the interleave16 gate||up columns), on each work-group tile."""
    qw, sc = weights(K, 2 * I, 8)
    x = O.f32_to_f16_bits(np.random.default_rng(8).standard_normal((T, K)).astype(np.float32))
    dq, ds, dx = dev(qw), dev(sc), dev(x)
    out = empty((T, 2 * I), np.float32)
    want = empty((T, I), np.uint16)
    got = empty((T, I), np.uint16)
    mi.call("mi_gemm_w4a16", ptr(dq), ptr(ds), ptr(dx), ptr(out), T, K, 2 * I, stream())
    mi.call("mi_silu_mul", ptr(out), ptr(want), T, I, 1, stream())
    mi.call("mi_gemm_w4a16_silu", ptr(dq), ptr(ds), ptr(dx), ptr(got), T, K, 2 * I, stream())
    sync()
    assert np.array_equal(host(got, np.uint16), host(want, np.uint16))


@pytest.mark.parametrize("QH,KVH,HD,rot,qk,paged", [(40, 8, 128, 128, True, False), (16, 2, 256, 64, False, True)])
def test_attn_prep_rows_is_attn_prep(QH, KVH, HD, rot, qk, paged):
    """mi_attn_prep_rows (one wave per head and row): bitwise mi_attn_prep on the same one-slice
    fold, for T rows at pos0 (attn_q and the written cache rows; the other rows untouched)."""
    sh = O.attn_shape(QH, KVH, HD, rot_dim=rot)
    T, pos0, Lm, P = 37, 100, 256, 64
    rng = np.random.default_rng(QH + HD)
    qkv = rng.standard_normal((T, sh.qkv_n)).astype(np.float32)
    qn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk else None
    kn = (1 + 0.05 * rng.standard_normal(HD)).astype(np.float32) if qk else None
    rope = O.rope_table(1e6, rot, Lm)
    pages = rng.permutation(Lm // P).astype(np.uint32) if paged else None
    kk = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    keep = [dev(qkv), dev(qn), dev(kn), dev(rope), dev(pages)]
    pp = [ptr(k) if k is not None else None for k in keep]
    c = np.zeros(64, np.uint32)
    c[0], c[1] = pos0, T
    ctrl = dev(c)
    q1, k1, v1 = empty((T, QH, HD), np.float32), dev(kk), dev(kk)
    q2, k2, v2 = empty((T, QH, HD), np.float32), dev(kk), dev(kk)
    print(f"attn_prep_rows {QH}/{KVH}x{HD}", flush=True)
    mi.call("mi_attn_prep", ptr(ctrl), pp[0], 1, T, mi.shape_ref(sh), pp[1], pp[2], pp[3], ptr(q1), None, ptr(k1),
            ptr(v1), HD, Lm * HD, pp[4], P if paged else 0, Lm, stream())
    mi.call("mi_attn_prep_rows", pp[0], T, pos0, mi.shape_ref(sh), pp[1], pp[2], pp[3], ptr(q2), ptr(k2), ptr(v2), HD,
            Lm * HD, pp[4], P if paged else 0, stream())
    sync()
    assert np.array_equal(host(q2, np.uint32), host(q1, np.uint32))
    assert np.array_equal(host(k2, np.uint16), host(k1, np.uint16))
    assert np.array_equal(host(v2, np.uint16), host(v1, np.uint16))


def test_gemm_refuses_bad_shapes():
    with pytest.raises(mi.MiError):
        mi.call("mi_gemm_w4a16", 16, 16, 16, 16, 4, 100, 128, None)
    with pytest.raises(mi.MiError):
        mi.call("mi_gemm_w4a16", 16, 16, 16, 16, 4, 128, 100, None)


def prefill_attention(sh, q, k, v, T, pos0, pages=None, page=0):
    HD, QH = sh.head_dim, sh.q_heads
    Lm = k.shape[1]
    dq, dk, dv, dpg = dev(q), dev(k), dev(v), dev(pages)
    out = empty((T, QH * HD), np.uint16)
    mi.call("mi_attn_prefill", ptr(dq), ptr(dk), ptr(dv), HD, Lm * HD, ptr(dpg), page, T, pos0, mi.shape_ref(sh),
            ptr(out), stream())
    sync()
    return host(out, np.uint16)


@pytest.mark.parametrize("QH,KVH,HD,T,pos0", [(40, 8, 128, 37, 100), (40, 8, 128, 130, 0), (16, 2, 256, 20, 64),
                                              (8, 8, 128, 65, 3)])
def test_attn_prefill_vs_fp64(QH, KVH, HD, T, pos0):
    sh = O.attn_shape(QH, KVH, HD)
    Lm = 256
    rng = np.random.default_rng(QH + T)
    k = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    v = O.f32_to_f16_bits(rng.standard_normal((KVH, Lm, HD)).astype(np.float32))
    q = rng.standard_normal((T, QH, HD)).astype(np.float32)
    print(f"attn_prefill {QH}/{KVH}x{HD} T={T} pos0={pos0}", flush=True)
    got = prefill_attention(sh, q, k, v, T, pos0)
    G = QH // KVH
    want = np.zeros((T, QH, HD))
    for t in range(T):
        for h in range(QH):
            O.lib().orc_attend64(C.byref(sh), O._p(np.ascontiguousarray(q[t, h])), h // G, pos0 + t + 1, 0, F16,
                                 O._p(k), O._p(v), None, None, HD, Lm * HD, 1, Lm, None, 0, O._p(want[t, h]))
    g = O.f16_bits_to_f32(got).astype(np.float64).reshape(T, QH, HD)
    err = np.abs(g - want)
    assert np.all(err <= 2e-3 * np.abs(want) + 2e-3 * np.abs(want).max(axis=-1, keepdims=True)), err.max()
    cos = (g * want).sum(-1) / np.sqrt((g * g).sum(-1) * (want * want).sum(-1))
    assert cos.min() >= 0.99999


def test_attn_prefill_paged_bitwise():
    sh = O.attn_shape(40, 8, 128)
    Lm, P, T, pos0 = 512, 64, 50, 300
    rng = np.random.default_rng(5)
    k = O.f32_to_f16_bits(rng.standard_normal((8, Lm, 128)).astype(np.float32))
    v = O.f32_to_f16_bits(rng.standard_normal((8, Lm, 128)).astype(np.float32))
    q = rng.standard_normal((T, 40, 128)).astype(np.float32)
    a = prefill_attention(sh, q, k, v, T, pos0)
    pages = rng.permutation(Lm // P).astype(np.uint32)
    phys = np.concatenate([np.arange(pg * P, pg * P + P) for pg in pages])
    kp, vp = np.empty_like(k), np.empty_like(v)
    kp[:, phys], vp[:, phys] = k, v
    b = prefill_attention(sh, q, kp, vp, T, pos0, pages, P)
    assert np.array_equal(a, b)


def kv_rows(eng, p0, n):
    d = eng.desc
    k = eng.to_host(mi.T_KV_K, 0, np.uint16).reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)
    v = eng.to_host(mi.T_KV_V, 0, np.uint16).reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)
    f = lambda a: O.f16_bits_to_f32(a[:, :, p0:p0 + n]).astype(np.float64)
    return f(k), f(v)


@pytest.mark.parametrize("n,chunk,p0", [(40, 0, 0), (40, 16, 0), (33, 8, 100)])
def test_prefill_matches_ingest(n, chunk, p0):
    eng = mi.Engine(small_desc(max_len=512), seed=11)
    eng.capture(1)
    ids = np.random.default_rng(n + chunk).integers(0, eng.desc.vocab_used, n).astype(np.uint32)
    print(f"prefill vs ingest n={n} chunk={chunk} p0={p0}", flush=True)
    eng.reset(p0, 0)
    eng.ingest(ids)
    c_ing = eng.ctrl()
    lg_ing = eng.logits(1)[0].astype(np.float64)
    k_ing, v_ing = kv_rows(eng, p0, n)
    eng.reset(p0, 0)
    eng.prefill(ids, chunk)
    c_pf = eng.ctrl()
    lg_pf = eng.logits(1)[0].astype(np.float64)
    k_pf, v_pf = kv_rows(eng, p0, n)
    assert c_pf[mi.CTRL_POS] == c_ing[mi.CTRL_POS] == p0 + n
    assert c_pf[mi.CTRL_NACT] == 1
    # the two paths differ by the f16 rounding of the dequantised weights (2^-11 relative each)
    for a, b in ((k_pf, k_ing), (v_pf, v_ing)):
        assert np.all(np.abs(a - b) <= 0.02 * np.abs(b) + 0.02 * np.abs(b).max()), np.abs(a - b).max()
    scale = np.abs(lg_ing).max()
    assert np.all(np.abs(lg_pf - lg_ing) <= 0.01 * scale), np.abs(lg_pf - lg_ing).max() / scale
    top2 = np.sort(lg_ing)[-2:]
    if top2[1] - top2[0] > 0.02 * scale:
        assert c_pf[mi.CTRL_CUR] == c_ing[mi.CTRL_CUR] == int(np.argmax(lg_ing))
    # decode continues from the prefilled cache as from the ingested one
    eng.close()


@pytest.mark.parametrize("n,chunk,p0,qk_norm", [(40, 0, 0, 1), (40, 16, 0, 1), (33, 8, 100, 0)])
def test_prefill_vs_oracle_prefill(n, chunk, p0, qk_norm):
    """The engine's chunked prefill against the oracle's prefill walk (orc_prefill_chunk, chunk by
    chunk on the same cache): the last position's logits and every K/V row written, at the
    north star's rel 2e-3, and the control block as ingest leaves it."""
    eng = mi.Engine(small_desc(max_len=512, qk_norm=qk_norm), seed=13)
    orc = OracleModel(eng)
    ids = np.random.default_rng(n + chunk + 1).integers(0, eng.desc.vocab_used, n).astype(np.uint32)
    print(f"prefill vs oracle n={n} chunk={chunk} p0={p0} qk_norm={qk_norm}", flush=True)
    eng.reset(p0, 0)
    eng.prefill(ids, chunk)
    c = eng.ctrl()
    lg = eng.logits(1)[0].astype(np.float64)
    k_pf, v_pf = kv_rows(eng, p0, n)
    step = chunk or n
    want = np.zeros(eng.desc.vocab, np.float32)
    for c0 in range(0, n, step):
        part = np.ascontiguousarray(ids[c0:c0 + step])
        am = O.lib().orc_prefill_chunk(O.ORC_F16, C.byref(orc.m), O._p(part), len(part), p0 + c0, O._p(orc.kv_k),
                                       O._p(orc.kv_v), O._p(want))
    d = eng.desc
    kw = orc.kv_k.reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)[:, :, p0:p0 + n]
    vw = orc.kv_v.reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)[:, :, p0:p0 + n]
    for a, b in ((k_pf, kw), (v_pf, vw)):
        b = O.f16_bits_to_f32(b).astype(np.float64)
        assert np.all(np.abs(a - b) <= 2e-3 * np.abs(b) + 2e-3 * np.abs(b).max()), np.abs(a - b).max()
    w = want.astype(np.float64)
    assert close(lg, w), np.abs(lg - w).max() / np.abs(w).max()
    assert c[mi.CTRL_POS] == p0 + n and c[mi.CTRL_NACT] == 1
    top2 = np.sort(w)[-2:]
    if top2[1] - top2[0] > 4e-3 * np.abs(w).max():
        assert c[mi.CTRL_CUR] == am
    eng.close()


def test_prefill_refusals():
    eng = mi.Engine(small_desc(max_len=256), seed=2)
    eng.reset(250, 0)
    with pytest.raises(mi.MiError):
        eng.prefill(np.arange(10, dtype=np.uint32))  # past the cache
    eng.reset(0, 0)
    with pytest.raises(mi.MiError):
        eng.prefill(np.array([eng.desc.vocab], np.uint32))  # outside the vocabulary
    with pytest.raises(mi.MiError):
        eng.prefill(np.arange(4, dtype=np.uint32), 4096)  # chunk above the cap
    eng.close()


def test_moe_prefill_matches_ingest():
    """A mixture-of-experts model: the expert kernels run over the chunk's rows in slices. Layer
    0's K/V rows come before any routing and hold the dense bar; later layers sit behind top-k
    routing, where a near-tied expert choice may flip between the two roundings, so the last
    logits are held to a cosine bar there."""
    from test_engine_gpu import moe_small_desc
    eng = mi.Engine(moe_small_desc(max_len=512), seed=12)
    eng.capture(1)
    n, p0 = 37, 20
    ids = np.random.default_rng(3).integers(0, eng.desc.vocab_used, n).astype(np.uint32)
    print(f"moe prefill vs ingest n={n} p0={p0}", flush=True)
    eng.reset(p0, 0)
    eng.ingest(ids)
    c_ing, lg_ing = eng.ctrl(), eng.logits(1)[0].astype(np.float64)
    k_ing, v_ing = kv_rows(eng, p0, n)
    eng.reset(p0, 0)
    eng.prefill(ids, 16)
    c_pf, lg_pf = eng.ctrl(), eng.logits(1)[0].astype(np.float64)
    k_pf, v_pf = kv_rows(eng, p0, n)
    assert c_pf[mi.CTRL_POS] == c_ing[mi.CTRL_POS] == p0 + n
    for a, b in ((k_pf[0], k_ing[0]), (v_pf[0], v_ing[0])):
        assert np.all(np.abs(a - b) <= 0.02 * np.abs(b) + 0.02 * np.abs(b).max()), np.abs(a - b).max()
    cos = (lg_pf * lg_ing).sum() / np.sqrt((lg_pf * lg_pf).sum() * (lg_ing * lg_ing).sum())
    assert cos >= 0.99, cos
    eng.close()


def test_moe_prefill_vs_oracle_prefill():
    """The MoE model's chunked prefill against the oracle's prefill walk (orc_prefill_chunk with
    the experts as orc_moe_prefill, pinned to pf_moe_ref.h): every K/V row and the last logits
    at rel 2e-3."""
    from test_engine_gpu import moe_small_desc
    eng = mi.Engine(moe_small_desc(max_len=512), seed=12)
    orc = OracleModel(eng)
    n, p0, chunk = 37, 20, 16
    ids = np.random.default_rng(3).integers(0, eng.desc.vocab_used, n).astype(np.uint32)
    print(f"moe prefill vs oracle n={n} p0={p0}", flush=True)
    eng.reset(p0, 0)
    eng.prefill(ids, chunk)
    lg = eng.logits(1)[0].astype(np.float64)
    k_pf, v_pf = kv_rows(eng, p0, n)
    want = np.zeros(eng.desc.vocab, np.float32)
    for c0 in range(0, n, chunk):
        part = np.ascontiguousarray(ids[c0:c0 + chunk])
        O.lib().orc_prefill_chunk(O.ORC_F16, C.byref(orc.m), O._p(part), len(part), p0 + c0, O._p(orc.kv_k),
                                  O._p(orc.kv_v), O._p(want))
    d = eng.desc
    kw = orc.kv_k.reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)[:, :, p0:p0 + n]
    vw = orc.kv_v.reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)[:, :, p0:p0 + n]
    for a, b in ((k_pf, kw), (v_pf, vw)):
        b = O.f16_bits_to_f32(b).astype(np.float64)
        assert np.all(np.abs(a - b) <= 2e-3 * np.abs(b) + 2e-3 * np.abs(b).max()), np.abs(a - b).max()
    w = want.astype(np.float64)
    assert close(lg, w), np.abs(lg - w).max() / np.abs(w).max()
    eng.close()


def test_attn_prefill_kv8_rows_match_the_decode_reader():
    """mi_attn_prefill_kv8 over the int8 rotated cache: row t equals the decode reader's
    (attn_decode int8 + attn_reduce_kv8, itself held to fp64 attention with an fp64
    un-rotation in test_kv8_gpu) at position pos0 + t, within rel 2e-3 / cosine 0.99999."""
    QH, KVH, HD, Lm, T, pos0 = 16, 2, 256, 256, 20, 64
    sh = O.attn_shape(QH, KVH, HD)
    rng = np.random.default_rng(31)
    k8 = rng.integers(-127, 128, size=(KVH, Lm, HD)).astype(np.int8)
    v8 = rng.integers(-127, 128, size=(KVH, Lm, HD)).astype(np.int8)
    ks = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, Lm)).astype(np.float32))
    vs = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, Lm)).astype(np.float32))
    q = rng.standard_normal((T, QH, HD)).astype(np.float32)
    dk, dv, dks, dvs, dq = dev(k8), dev(v8), dev(ks), dev(vs), dev(q)
    rot = empty((T, QH, HD), np.float32)
    out = empty((T, QH * HD), np.uint16)
    print("attn_prefill_kv8", flush=True)
    mi.call("mi_attn_prefill_kv8", ptr(dq), ptr(dk), ptr(dv), ptr(dks), ptr(dvs), HD, Lm * HD, 1, Lm, None, 0, T,
            pos0, mi.shape_ref(sh), ptr(rot), ptr(out), stream())
    sync()
    got = O.f16_bits_to_f32(host(out, np.uint16)).astype(np.float64).reshape(T, QH, HD)
    tgt = 16
    for t in (0, 7, T - 1):
        c = np.zeros(64, np.uint32)
        c[0], c[1] = pos0 + t, 1
        ctrl = dev(c)
        qt = dev(np.ascontiguousarray(q[t:t + 1]))
        part = empty((QH, tgt, 1, HD + 2), np.float32)
        want16 = empty((1, QH * HD), np.uint16)
        mi.call("mi_attn_decode", ptr(ctrl), ptr(qt), 1, ptr(dk), ptr(dv), ptr(dks), ptr(dvs), HD, Lm * HD, 1, Lm,
                None, 0, Lm, ptr(part), 1, tgt, mi.shape_ref(sh), stream())
        mi.call("mi_attn_reduce_kv8", ptr(ctrl), ptr(part), None, ptr(want16), 1, tgt, Lm, mi.shape_ref(sh), stream())
        sync()
        want = O.f16_bits_to_f32(host(want16, np.uint16)).astype(np.float64).reshape(QH, HD)
        g = got[t]
        err = np.abs(g - want)
        assert np.all(err <= 2e-3 * np.abs(want) + 2e-3 * np.abs(want).max(axis=-1, keepdims=True)), (t, err.max())
        cos = (g * want).sum(-1) / np.sqrt((g * g).sum(-1) * (want * want).sum(-1))
        assert cos.min() >= 0.99999, t


def test_int8_cache_prefill_matches_ingest():
    eng = mi.Engine(small_desc(max_len=256, head_dim=256, q_heads=8, kv_heads=2, kv_int8=1), seed=13)
    eng.capture(1)
    d = eng.desc
    n, p0 = 30, 10
    ids = np.random.default_rng(9).integers(0, d.vocab_used, n).astype(np.uint32)
    print(f"int8-cache prefill vs ingest n={n} p0={p0}", flush=True)

    def rows():
        k = eng.to_host(mi.T_KV_K, 0, np.int8).reshape(d.layers, d.kv_heads, d.max_len, d.head_dim)
        ks = O.f16_bits_to_f32(eng.to_host(mi.T_KV_KS, 0, np.uint16).reshape(d.layers, d.kv_heads, d.max_len))
        return k[:, :, p0:p0 + n].astype(np.float64) * ks[:, :, p0:p0 + n, None]

    eng.reset(p0, 0)
    eng.ingest(ids)
    c_ing, lg_ing, k_ing = eng.ctrl(), eng.logits(1)[0].astype(np.float64), rows()
    eng.reset(p0, 0)
    eng.prefill(ids, 16)
    c_pf, lg_pf, k_pf = eng.ctrl(), eng.logits(1)[0].astype(np.float64), rows()
    assert c_pf[mi.CTRL_POS] == c_ing[mi.CTRL_POS] == p0 + n
    assert np.all(np.abs(k_pf - k_ing) <= 0.03 * np.abs(k_ing).max()), np.abs(k_pf - k_ing).max()
    scale = np.abs(lg_ing).max()
    assert np.all(np.abs(lg_pf - lg_ing) <= 0.01 * scale), np.abs(lg_pf - lg_ing).max() / scale
    eng.close()

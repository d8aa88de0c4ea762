"""The oracle pinned WITHOUT the reference build: the reference's committed golden
fixtures, its tests' known answers, and what the mathematics fixes (closed forms, fp64
brute force, exact-arithmetic cases). CPU only."""
import os

import numpy as np
import pytest

import oracle as O
import safetensors_raw

GOLD = os.path.join(os.path.dirname(__file__), "golden")
L = O.lib


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


# ---- conversions -------------------------------------------------------------------------
def test_f16_widen_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([L().orc_f16_to_f32(int(v)) for v in h], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    assert np.all(np.isnan(got[~fin]) == np.isnan(want[~fin]))


def test_f32_to_f16_rne_matches_ieee():
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1e-5, 5.96e-8, 2.98e-8,
                  2.99e-8, 1e-10], np.float32)])
    want = vals.astype(np.float16).view(np.uint16)
    got = np.array([L().orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


def test_rne_ties_known_answers():
    # tests/kernels/int4_test.cc:17-31: exact ties go to the even neighbour
    f = lambda u: np.array([u], np.uint32).view(np.float32)[0]
    assert L().orc_f32_to_bf16(float(f(0x3F808000))) == 0x3F80
    assert L().orc_f32_to_bf16(float(f(0x3F818000))) == 0x3F82
    assert L().orc_f32_to_f16(float(f((127 << 23) | (1 << 13) | 0x1000))) == 0x3C02
    assert L().orc_f32_to_f16(float(f((127 << 23) | 0x1000))) == 0x3C00
    assert L().orc_f32_to_bf16(1.0) == 0x3F80
    assert L().orc_f16_to_f32(0x3C00) == 1.0


# ---- int4 --------------------------------------------------------------------------------
def test_dequant_fixture_bit_exact():
    """tests/golden/dequant_fixture.safetensors (written by the reference's tools/oracle/
    dequant.py, seed 1234): rne_bf16 of the oracle's dequant equals it element for element."""
    t = safetensors_raw.load(os.path.join(GOLD, "dequant_fixture.safetensors"))
    qw = np.ascontiguousarray(t["qweight"][1].view(np.uint32))
    sc = _u16(t["scales"][1])
    gold = t["dequant"][1]
    K, N = qw.shape[0] * 8, qw.shape[1]
    deq = O.int4_dequant(qw, sc, K, N)
    assert np.array_equal(O.f32_to_bf16_bits(deq), gold)


def test_int4_known_answers():
    """tests/kernels/int4_test.cc:33-48: nibble order, group index."""
    K, N = 128, 16
    qw = np.zeros((K // 8, N), np.uint32)
    sc = np.full((K // 64, N), 0x3800, np.uint16)  # 0.5
    sc[1, :] = 0x3400                               # 0.25
    qw[0, 3] = 0x0000000F
    qw[1, 3] = 0x00000080
    qw[9, 3] = 0xF << 12
    d = O.int4_dequant(qw, sc, K, N)
    assert d[0, 3] == 3.5 and d[1, 3] == -4.0 and d[9, 3] == 0.0
    assert d[75, 3] == 1.75 and d[74, 3] == -2.0


def test_int4_exhaustive_nibbles():
    """Every nibble value at every position of a word, against (q - 8) * scale."""
    K, N = 64, 16
    qw = np.zeros((K // 8, N), np.uint32)
    for r in range(K // 8):
        for n in range(N):
            qw[r, n] = sum(((r * 8 + i + n) % 16) << (4 * i) for i in range(8))
    sc = np.full((1, N), 0x3C00, np.uint16)
    d = O.int4_dequant(qw, sc, K, N)
    for k in range(K):
        for n in range(N):
            assert d[k, n] == float(((k + n) % 16) - 8)


def test_interleave16_map():
    """tests/kernels/int4_test.cc:50-79's tagged values through the Interleave16 map."""
    RK, PN = 64, 32
    row = np.arange(RK // 8, dtype=np.uint32)[:, None]
    n = np.arange(PN, dtype=np.uint32)[None, :]
    aq = (0xA0000000 | (row << 8) | n).astype(np.uint32)
    bq = (0xB0000000 | (row << 8) | n).astype(np.uint32)
    as_ = (0x1000 + np.arange(PN)).astype(np.uint16)[None, :]
    bs = (0x2000 + np.arange(PN)).astype(np.uint16)[None, :]
    oq = np.zeros((RK // 8, 2 * PN), np.uint32)
    os_ = np.zeros((1, 2 * PN), np.uint16)
    L().orc_interleave16_l0(O._p(aq), O._p(np.ascontiguousarray(as_)), O._p(bq),
                            O._p(np.ascontiguousarray(bs)), RK, PN, O._p(oq), O._p(os_))
    for c in range(2 * PN):
        from_b = c % 32 >= 16
        src = (c // 32) * 16 + c % 16
        assert os_[0, c] == (0x2000 if from_b else 0x1000) + src
        for r in range(RK // 8):
            assert oq[r, c] == ((0xB0000000 if from_b else 0xA0000000) | (r << 8) | src)


def _rand_w(K, N, seed, lo=0.002, hi=0.02):
    rng = np.random.default_rng(seed)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = O.f32_to_f16_bits(rng.uniform(lo, hi, size=(K // 64, N)).astype(np.float32))
    return qw, sc


def test_layout1_same_values_and_order():
    """Layout 1 tiles hold the same (q, scale) per (k, n): the twin GEMV over the tiles is
    bitwise the twin over layout 0 (same values in the same order)."""
    K, N = 256, 64
    qw, sc = _rand_w(K, N, 3)
    tiles = np.zeros((N // 16) * (K // 64) * 136, np.uint32)
    L().orc_repack_layout1(O._p(qw), O._p(sc), K, N, O._p(tiles))
    x = np.random.default_rng(4).standard_normal(K).astype(np.float32)
    a = O.gemv_twin(qw, sc, K, N, x, S=2, layout=0)
    b = O.gemv_twin(tiles, None, K, N, x, S=2, layout=1)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- GEMV --------------------------------------------------------------------------------
@pytest.mark.parametrize("S", [1, 2, 4])
def test_gemv_twin_within_n2_of_fp64(S):
    K, N = 1024, 256
    qw, sc = _rand_w(K, N, 11)
    x = O.widen(O.ORC_F16, O.f32_to_f16_bits(np.random.default_rng(5).standard_normal((2, K))))
    ref, bound = O.gemv_ref(qw, sc, K, N, x)
    got = O.gemv_twin(qw, sc, K, N, x, S=S)
    over, mr = O.n2_over(got, ref, bound)
    assert over == 0, mr
    # an independent fp64 dequant-and-dot pins the fp64 reference itself
    W = O.int4_dequant(qw, sc, K, N).astype(np.float64)
    assert np.allclose(ref, x.astype(np.float64) @ W, rtol=0, atol=1e-9)


def test_gemv_exact_arithmetic():
    """Small-integer activations and power-of-two scales make every product and sum exact,
    so the twin must equal the integer result bit for bit (pins nibble order + groups)."""
    K, N = 512, 64
    rng = np.random.default_rng(9)
    qw = rng.integers(0, 2**32, size=(K // 8, N), dtype=np.uint64).astype(np.uint32)
    sc = rng.choice(np.array([0x3C00, 0x3800, 0x4000, 0x3400], np.uint16), size=(K // 64, N))
    x = rng.integers(-4, 5, size=K).astype(np.float32)
    W = O.int4_dequant(qw, sc, K, N).astype(np.float64)
    exact = x.astype(np.float64) @ W
    for S in (1, 4, 8):
        got = O.gemv_twin(qw, sc, K, N, x, S=S)[0]
        assert np.array_equal(got.astype(np.float64), exact)


# ---- prep --------------------------------------------------------------------------------
@pytest.mark.parametrize("act", [O.ORC_F16, O.ORC_BF16])
def test_res_norm_closed_form(act):
    M, K, S = 2, 5120, 4
    rng = np.random.default_rng(1)
    partials = (rng.standard_normal((S, M, K)) * 0.3).astype(np.float32)
    resid = O.rne(act, rng.standard_normal((M, K)).astype(np.float32))
    w = (1 + 0.02 * rng.standard_normal(K)).astype(np.float32)
    r2, x = O.res_norm(act, partials, resid, w, M, K, S)
    # the residual: rne(resid + rne(sum_s partials)) with the sum in s order
    fold = np.zeros((M, K), np.float32)
    for s in range(S):
        fold = fold + partials[s]
    want_r = O.rne(act, O.widen(act, resid) + O.widen(act, O.rne(act, fold)))
    assert np.array_equal(r2, want_r)
    rf = O.widen(act, r2).astype(np.float64)
    rstd = 1.0 / np.sqrt((rf ** 2).mean(axis=1, keepdims=True) + 1e-6)
    want = rf * rstd * w
    got = O.widen(act, x).astype(np.float64)
    ulp = 2.0 ** -10 if act == O.ORC_F16 else 2.0 ** -7
    assert np.all(np.abs(got - want) <= ulp * np.abs(want) + 1e-30)
    # S_PREV = 0 leaves the residual as it was
    r3, _ = O.res_norm(act, None, resid, w, M, K, 0)
    assert np.array_equal(r3, resid)


def test_silu_mul_exp_free_point_and_fp64():
    act, M, N, S = O.ORC_F16, 1, 512, 2
    rng = np.random.default_rng(2)
    part = (rng.standard_normal((S, M, 2 * N)) * 2).astype(np.float32)
    gcol = lambda k: (k // 16) * 32 + k % 16
    # x = 30: exp(-30) vanishes next to 1 in fp32, so silu(30) = 30 exactly
    part[:, 0, gcol(5)] = [30.0, 0.0]
    x = O.silu_mul(act, part, M, N, S)
    g = np.array([part[:, 0, gcol(k)].sum(dtype=np.float32) for k in range(N)], np.float32)
    u = np.array([part[:, 0, gcol(k) + 16].sum(dtype=np.float32) for k in range(N)], np.float32)
    gb = O.widen(act, O.rne(act, g)).astype(np.float64)
    ub = O.widen(act, O.rne(act, u)).astype(np.float64)
    assert O.widen(act, x[0, 5:6])[0] == O.widen(act, O.rne(act, np.float32(30.0 * ub[5])))
    sb = O.widen(act, O.rne(act, (gb / (1 + np.exp(-gb))).astype(np.float32))).astype(np.float64)
    want = sb * ub
    got = O.widen(act, x[0]).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2 * 2.0 ** -10 * np.abs(want) + 1e-7)


# ---- attention ---------------------------------------------------------------------------
def _attn_setup(act, L_, QH=8, KVH=2, HD=128, seed=0, kv_kind=0):
    rng = np.random.default_rng(seed)
    sh = O.attn_shape(QH, KVH, HD)
    q = rng.standard_normal((1, QH, HD)).astype(np.float32)
    if kv_kind == 0:
        k = O.rne(act, rng.standard_normal((KVH, L_, HD)).astype(np.float32))
        v = O.rne(act, rng.standard_normal((KVH, L_, HD)).astype(np.float32))
        ks = vs = None
    else:
        k = rng.integers(-127, 128, size=(KVH, L_, HD)).astype(np.int8)
        v = rng.integers(-127, 128, size=(KVH, L_, HD)).astype(np.int8)
        ks = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, L_)).astype(np.float32))
        vs = O.f32_to_f16_bits(rng.uniform(0.005, 0.05, (KVH, L_)).astype(np.float32))
    return sh, q, k, v, ks, vs


def _decode(act, sh, q, k, v, ks, vs, pos, tgt, kv_kind=0, pages=None, page=0):
    QH, HD, L_ = sh.q_heads, sh.head_dim, k.shape[1]
    part = np.zeros((QH, tgt, 1, HD + 2), np.float32)
    L().orc_attn_decode_v2(act, O.C.byref(sh), pos, 1, 1, tgt, O._p(q), kv_kind, O._p(k), O._p(v),
                           O._p(ks), O._p(vs), HD, L_ * HD, 1, L_, O._p(pages), page, O._p(part))
    out = np.zeros((1, QH * HD), np.uint16)
    L().orc_attn_reduce_v2(act, O.C.byref(sh), pos, 1, 1, tgt, O._p(part), None, O._p(out))
    return out, part


@pytest.mark.parametrize("kv_kind", [0, 1])
@pytest.mark.parametrize("pos", [0, 15, 200, 3000])
def test_attention_v2_vs_fp64(kv_kind, pos):
    act = O.ORC_F16
    L_ = 4096
    sh, q, k, v, ks, vs = _attn_setup(act, L_, kv_kind=kv_kind, seed=pos)
    out, _ = _decode(act, sh, q, k, v, ks, vs, pos, 32, kv_kind)
    got = O.widen(act, out[0]).reshape(sh.q_heads, sh.head_dim).astype(np.float64)
    for h in range(sh.q_heads):
        o = np.zeros(sh.head_dim, np.float64)
        L().orc_attend64(O.C.byref(sh), O._p(np.ascontiguousarray(q[0, h])), h // 4, pos + 1, kv_kind,
                         act, O._p(k), O._p(v), O._p(ks), O._p(vs), sh.head_dim, L_ * sh.head_dim, 1,
                         L_, None, 0, O._p(o))
        # independent numpy softmax attention
        kk = O.widen(act, k[h // 4, :pos + 1]) if kv_kind == 0 else \
            k[h // 4, :pos + 1].astype(np.float64) * O.f16_bits_to_f32(ks[h // 4, :pos + 1])[:, None]
        vv = O.widen(act, v[h // 4, :pos + 1]) if kv_kind == 0 else \
            v[h // 4, :pos + 1].astype(np.float64) * O.f16_bits_to_f32(vs[h // 4, :pos + 1])[:, None]
        sc = kk.astype(np.float64) @ q[0, h].astype(np.float64) * float(sh.scale)
        p = np.exp(sc - sc.max())
        want = (p / p.sum()) @ vv.astype(np.float64)
        assert np.allclose(o, want, rtol=1e-12, atol=1e-12)
        assert np.all(np.abs(got[h] - want) <= 2e-3 * np.abs(want).max() + 1e-3 * np.abs(want))


def test_attention_paged_bitwise_contiguous():
    act, L_, P = O.ORC_F16, 2048, 64
    for kv_kind in (0, 1):
        sh, q, k, v, ks, vs = _attn_setup(act, L_, kv_kind=kv_kind, seed=3)
        rng = np.random.default_rng(4)
        pages = rng.permutation(L_ // P).astype(np.uint32)
        # scatter logical rows into physical rows through the table
        phys = np.concatenate([np.arange(pg * P, pg * P + P) for pg in pages])
        kp, vp = np.empty_like(k), np.empty_like(v)
        kp[:, phys], vp[:, phys] = k, v
        ksp = vsp = None
        if kv_kind:
            ksp, vsp = np.empty_like(ks), np.empty_like(vs)
            ksp[:, phys], vsp[:, phys] = ks, vs
        for pos in (0, 63, 64, 1500, 2047):
            a, pa = _decode(act, sh, q, k, v, ks, vs, pos, 16, kv_kind)
            b, pb = _decode(act, sh, q, kp, vp, ksp, vsp, pos, 16, kv_kind, pages, P)
            assert np.array_equal(a, b) and np.array_equal(pa.view(np.uint32), pb.view(np.uint32))


def test_attn_prep_rope_closed_form():
    """q/k RMSNorm + RoPE + KV write against a float64 restatement of the maths (the RoPE
    table from the formula, the rotate_half pairs); V is the linear's rounding, exactly."""
    act, QH, KVH, HD, S, pos, Lm = O.ORC_F16, 4, 2, 128, 2, 37, 64
    sh = O.attn_shape(QH, KVH, HD)
    rng = np.random.default_rng(6)
    part = rng.standard_normal((S, 1, sh.qkv_n)).astype(np.float32)
    qn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    kn = (1 + 0.02 * rng.standard_normal(HD)).astype(np.float32)
    rope = O.rope_table(1e6, HD, Lm)
    half = HD // 2
    inv = 1e6 ** (-2.0 * np.arange(half) / HD)
    assert np.allclose(rope[pos, 0], np.cos(pos * inv), atol=1e-7)
    assert np.allclose(rope[pos, 1], np.sin(pos * inv), atol=1e-7)
    aq = np.zeros((1, QH, HD), np.float32)
    kk = np.zeros((KVH, Lm, HD), np.uint16)
    vv = np.zeros((KVH, Lm, HD), np.uint16)
    L().orc_attn_prep(act, O.C.byref(sh), pos, 1, 1, O._p(part), S, O._p(qn), O._p(kn), O._p(rope),
                      O._p(aq), None, O._p(kk), O._p(vv), HD, Lm * HD, None, 0)
    lin = part.sum(axis=0, dtype=np.float32)[0]
    lin_b = O.widen(act, O.rne(act, lin)).astype(np.float64)

    def normed_roped(col0, w):
        x = lin_b[col0:col0 + HD]
        n = x / np.sqrt((x ** 2).mean() + 1e-6) * w
        c, s = np.cos(pos * inv), np.sin(pos * inv)
        return np.concatenate([n[:half] * c - n[half:] * s, n[half:] * c + n[:half] * s])

    for h in range(QH):
        want = normed_roped(h * HD, qn)
        assert np.allclose(aq[0, h], want, rtol=0, atol=4e-3 * np.abs(want).max())
    for h in range(KVH):
        want = normed_roped(sh.k_off + h * HD, kn)
        got = O.widen(act, kk[h, pos]).astype(np.float64)
        assert np.allclose(got, want, rtol=0, atol=4e-3 * np.abs(want).max())
        assert np.array_equal(vv[h, pos], O.rne(act, lin[sh.v_off + h * HD:sh.v_off + (h + 1) * HD]))
        assert not vv[h, pos + 1].any()


# ---- int8 KV (the reference's rotkv scheme) ------------------------------------------------
def test_kv8_sim_fixture_bitwise():
    """tests/golden/kv8_sim_fixture.safetensors (the reference's int8_sim.py rows): codes,
    fp16 scales and dequantised values bit for bit, xhat = fp32(fp64 unrotate(deq))."""
    t = safetensors_raw.load(os.path.join(GOLD, "kv8_sim_fixture.safetensors"))
    x = O.bf16_bits_to_f32(t["x"][1])
    R = x.shape[0]
    signs = np.array([(w >> b) & 1 for w in [0xA197D809, 0xA6850592, 0xB205A73E, 0x20AFA769,
                                             0x45C2CF64, 0xBEAEAACB, 0x75F39ADD, 0x2385A70C]
                      for b in range(32)], bool)

    def fwht64(v):  # the canonical in-place FWHT, stages h = 1, 2, ..., 128, in float64
        v = v.copy()
        h = 1
        while h < 256:
            v = v.reshape(-1, 2, h)
            a, c = v[:, 0, :].copy(), v[:, 1, :].copy()
            v[:, 0, :], v[:, 1, :] = a + c, a - c
            v = v.reshape(256)
            h *= 2
        return v
    for r in range(R):
        q = np.zeros(256, np.int8)
        row = np.ascontiguousarray(x[r])
        s = L().orc_kv8_encode256(O._p(row), O._p(q))
        assert s == t["s16"][1][r]
        assert np.array_equal(q, t["q"][1][r])
        deq = np.array([L().orc_kv8_dequant(int(c), s) for c in q], np.float32)
        assert np.array_equal(deq.view(np.uint32), t["deq"][1][r].view(np.uint32))
        v = np.where(signs, -deq.astype(np.float64), deq.astype(np.float64))
        xhat = (fwht64(v) * 0.0625).astype(np.float32)
        assert np.array_equal(xhat.view(np.uint32), t["xhat"][1][r].view(np.uint32))


# ---- token boundary ------------------------------------------------------------------------
def test_argmax_known_answers():
    """tests/kernels/argmax_test.cc:93-130's cases, at this vocabulary (151936, all usable
    ids but a masked tail of 100 for the tail case)."""
    V = 151936
    rng = lambda s: np.random.default_rng(s).uniform(-4, -1, V).astype(np.float32)
    v = rng(11); v[123456] = 3.5
    assert O.argmax(v) == 123456
    v = rng(12); v[5000] = v[5001] = v[90000] = 7.0
    assert O.argmax(v) == 5000
    v = rng(13); v[V - 100] = 99.0; v[V - 20] = 100.0; v[1000] = 42.0
    assert O.argmax(v, V - 100) == 1000
    assert O.argmax(np.zeros(V, np.float32)) == 0
    v = rng(14); v[V - 1] = 5.0
    assert O.argmax(v) == V - 1
    v = rng(15)
    assert O.argmax(v) == int(np.argmax(v))


def test_accept_greedy_known_answers():
    """tests/server/spec_accept_test.cc:246-262."""
    am = [7, 8, 9, 10]
    assert O.accept_greedy(am, [7, 8, 9]) == (3, 10)
    assert O.accept_greedy(am, [1, 8, 9]) == (0, 7)
    assert O.accept_greedy(am, [7, 2, 9]) == (1, 8)
    assert O.accept_greedy(am, []) == (0, 7)


def test_embed_gather_and_bad_id():
    V, H = 64, 256
    emb = np.random.default_rng(0).integers(0, 65535, (V, H)).astype(np.uint16)
    out = np.full((2, H), 7, np.uint16)
    ids = np.array([5, 63], np.uint32)
    assert L().orc_embed_gather(O._p(ids), 2, O._p(emb), V, H, O._p(out)) == 0
    assert np.array_equal(out, emb[[5, 63]])
    out2 = np.full((1, H), 7, np.uint16)
    bad = np.array([V], np.uint32)
    assert L().orc_embed_gather(O._p(bad), 1, O._p(emb), V, H, O._p(out2)) & 0xFFFFFFFF == 0xDEAD0001
    assert np.all(out2 == 7)


# ---- MoE -----------------------------------------------------------------------------------
def _route(act, logits, E, K):
    r = O.MoeRoute()
    lg = np.ascontiguousarray(logits, np.float32)
    L().orc_moe_route_fn(act, O._p(lg), E, K, O.C.byref(r))
    return r


def test_moe_route_ties_known_answers():
    """tests/kernels/moe_ref_test.cc:40-78 (bf16, 16 experts, top-4)."""
    act, E, K = O.ORC_BF16, 16, 4
    lg = np.zeros(32, np.float32)
    lg[:E] = -4.0 + 0.25 * ((np.arange(E) * 7) % 16)
    lg[12] = lg[2] = 3.0
    lg[5] = 2.5
    lg[3] = lg[9] = 2.0
    lg[E] = 0.75
    r = _route(act, lg, E, K)
    assert list(r.ids[:4]) == [2, 12, 5, 3]
    assert r.p[0] == r.p[1] and r.p9 == r.p[3]
    sig = np.float32(1) / (np.float32(1) + np.exp(np.float32(-0.75)))
    assert r.sg == O.widen(act, O.rne(act, sig))
    eq = np.ones(32, np.float32)
    re = _route(act, eq, E, K)
    assert list(re.ids[:4]) == [0, 1, 2, 3]
    assert all(w == O.widen(act, O.rne(act, np.float32(0.25))) for w in re.w[:4])


def test_moe_combine_slot_order():
    """tests/kernels/moe_ref_test.cc:82-106: the fixed ascending slot order decides."""
    act = O.ORC_BF16
    tiny = np.float32(2.0 ** -15)
    for d in ([1024.0, tiny, -1024.0, tiny, 0, 0, 0, 0, 0], [0, 0, 0, 0, 1024.0, tiny, -1024.0, tiny, 0]):
        r = O.MoeRoute()
        for k in range(8):
            r.w[k] = 1.0
        r.sg = 0.0
        dd = np.array(d, np.float32)
        out = L().orc_moe_combine(act, O._p(dd), O.C.byref(r), 8, 0)
        assert out == O.rne(act, tiny)


def test_moe_block_vs_fp64():
    """tests/kernels/moe_ref_test.cc:139-258's independent double-precision MoE (softmax,
    stable sort, renormalise, dequantised experts, shared expert by its gate, residual)."""
    act, E, K, Hd, I = O.ORC_F16, 32, 4, 256, 128
    rng = np.random.default_rng(2026)
    gu = [None] * (E + 1)
    dn = [None] * (E + 1)
    for b in range(E + 1):
        gq, gs = _rand_w(Hd, I, 100 + 3 * b, 0.02, 0.08)
        uq, us = _rand_w(Hd, I, 101 + 3 * b, 0.02, 0.08)
        oq = np.zeros((Hd // 8, 2 * I), np.uint32)
        os_ = np.zeros((Hd // 64, 2 * I), np.uint16)
        L().orc_interleave16_l0(O._p(gq), O._p(gs), O._p(uq), O._p(us), Hd, I, O._p(oq), O._p(os_))
        gu[b] = (gq, gs, uq, us, oq, os_)
        dn[b] = _rand_w(I, Hd, 102 + 3 * b, 0.02, 0.08)
    guq = np.ascontiguousarray(np.stack([g[4] for g in gu]))
    gus = np.ascontiguousarray(np.stack([g[5] for g in gu]))
    dnq = np.ascontiguousarray(np.stack([d[0] for d in dn]))
    dns = np.ascontiguousarray(np.stack([d[1] for d in dn]))
    rf = lambda f: O.widen(act, O.rne(act, np.float32(f))).astype(np.float64)
    worst = 0
    for tok in range(3):
        x = O.rne(act, rng.uniform(-0.08, 0.08, Hd).astype(np.float32))
        resid = O.rne(act, rng.uniform(-3, 3, Hd).astype(np.float32)) if tok % 2 == 0 else np.zeros(Hd, np.uint16)
        logits = np.zeros(48, np.float32)
        logits[:E + 1] = rng.uniform(-3, 3, E + 1)
        r = _route(act, logits, E, K)
        got = resid.copy()
        L().orc_moe_block(act, 0, E, K, Hd, I, O.C.byref(r), O._p(x), O._p(guq), O._p(gus), guq[0].size,
                          gus[0].size, O._p(dnq), O._p(dns), dnq[0].size, dns[0].size, 2, 1, None, O._p(got))
        # naive double MoE
        lb = np.array([rf(v) for v in logits[:E]])
        p = np.exp(lb - lb.max()); p /= p.sum()
        ids = sorted(range(E), key=lambda e: (-p[e], e))[:K]
        assert list(r.ids[:K]) == ids
        xf = O.widen(act, x).astype(np.float64)

        def expert(b):
            gq, gs, uq, us = gu[b][:4]
            Wg = O.int4_dequant(gq, gs, Hd, I).astype(np.float64)
            Wu = O.int4_dequant(uq, us, Hd, I).astype(np.float64)
            g = np.array([rf(v) for v in xf @ Wg]); u = np.array([rf(v) for v in xf @ Wu])
            s = np.array([rf(v) for v in g / (1 + np.exp(-g))])
            h = np.array([rf(v) for v in s * u])
            Wd = O.int4_dequant(dn[b][0], dn[b][1], I, Hd).astype(np.float64)
            return np.array([rf(v) for v in h @ Wd])
        outs = [expert(e) for e in ids]
        sh = expert(E)
        ps = sum(p[e] for e in ids)
        sg = rf(1 / (1 + np.exp(-rf(logits[E]))))
        want = np.zeros(Hd, np.uint16)
        for n in range(Hd):
            s = sum(rf(outs[k][n] * rf(p[ids[k]] / ps)) for k in range(K))
            o = rf(rf(s) + rf(sh[n] * sg))
            want[n] = O.rne(act, np.float32(O.widen(act, resid[n:n + 1])[0] + o))
        a = O.widen(act, got).astype(np.float64)
        b_ = O.widen(act, want).astype(np.float64)
        ulp = np.maximum(np.abs(b_), 2.0 ** -14) * 2.0 ** -10
        worst = max(worst, float(np.max(np.abs(a - b_) / ulp)))
    assert worst <= 2.0


def _f16w_tiled(w_rm, K, N):
    wt = np.empty(K * N, np.uint16)
    O.lib().orc_f16w_tile(O._p(np.ascontiguousarray(w_rm)), K, N, O._p(wt))
    return wt


def test_gemv_f16w_merge_order_known_answer():
    """gemv_bf16.cl:37-41 documents the KSPLIT merge: at KSPLIT = 4 the column sum is
    (p0 + p2) + (p1 + p3). Slices 2^24, 1, -2^24, 1 give 2 that way; an ascending chain or an
    adjacent-pair tree gives 1."""
    K, N = 32, 16
    w = np.zeros((N, K), np.float32)
    x = np.zeros(K, np.float32)
    for q, (wv, xv) in enumerate([(4096.0, 4096.0), (1.0, 1.0), (-4096.0, 4096.0), (1.0, 1.0)]):
        w[:, 8 * q] = wv
        x[8 * q] = xv
    wt = _f16w_tiled(O.f32_to_f16_bits(w), K, N)
    out = np.empty(N, np.float32)
    O.lib().orc_gemv_f16w(O.ORC_F16, O._p(wt), O._p(O.f32_to_f16_bits(x)), 1, K, N, 4, O._p(out))
    assert np.all(out == 2.0)
    O.lib().orc_gemv_f16w(O.ORC_F16, O._p(wt), O._p(O.f32_to_f16_bits(x)), 1, K, N, 1, O._p(out))
    assert np.all(out == 1.0)


@pytest.mark.parametrize("ksplit", [1, 4, 16])
def test_gemv_f16w_vs_fp64(ksplit):
    """Router || shared-gate GEMV at config 4's shape (K 2048, N 272, M 2): within the
    sequential fp32 bound (K/ksplit + log2 ksplit) 2^-24 sum|w x| of fp64."""
    K, N, M = 2048, 272, 2
    rng = np.random.default_rng(ksplit)
    w = O.f32_to_f16_bits((0.02 * rng.standard_normal((N, K))).astype(np.float32))
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    out = np.empty((M, N), np.float32)
    O.lib().orc_gemv_f16w(O.ORC_F16, O._p(_f16w_tiled(w, K, N)), O._p(x), M, K, N, ksplit, O._p(out))
    wf = O.f16_bits_to_f32(w).astype(np.float64)
    xf = O.f16_bits_to_f32(x).astype(np.float64)
    want = xf @ wf.T
    bound = (K / ksplit + np.log2(ksplit) + 1) * 2.0 ** -24 * (np.abs(xf) @ np.abs(wf).T)
    assert np.all(np.abs(out - want) <= bound)


def test_int8_head_quantiser_known_answers():
    """lm_head_int8_test's hand-made rows: max 127 gives s = 1 exactly, so w / s is w and the
    ties are exact (2.5 -> 2, 3.5 -> 4, -2.5 -> -2, 0.5 -> 0, 1.5 -> 2, -0.5 -> 0, round to
    nearest even); a zero row gives s = 0 and q = 0; values past the row's scale clamp at
    +-127; the round trip |w - q s| <= s / 2 (1 + 2^-22)."""
    w = np.zeros(64, np.float32)
    w[:8] = [127.0, 2.5, 3.5, -2.5, -127.0, 0.5, 1.5, -0.5]
    q = np.zeros(64, np.int8)
    assert O.lib().orc_quantise_row_int8(O._p(w), 64, O._p(q)) == 1.0
    assert list(q[:8]) == [127, 2, 4, -2, -127, 0, 2, 0] and not np.any(q[8:])
    z = np.zeros(64, np.float32)
    qz = np.ones(64, np.int8)
    assert O.lib().orc_quantise_row_int8(O._p(z), 64, O._p(qz)) == 0.0 and not np.any(qz)
    rng = np.random.default_rng(3)
    r = (0.02 * rng.standard_normal(5120)).astype(np.float32)
    qr = np.zeros(5120, np.int8)
    s = O.lib().orc_quantise_row_int8(O._p(r), 5120, O._p(qr))
    assert s == np.float32(np.abs(r).max()) / np.float32(127.0)
    assert np.abs(qr.astype(np.int32)).max() == 127
    err = np.abs(r.astype(np.float64) - qr.astype(np.float64) * s)
    assert err.max() <= s * 0.5 * (1 + 2.0 ** -22)


def test_int8_gemv_vs_fp64():
    """orc_gemv_i8w (one fp32 chain over k, then the scale) within the fp32 summation bound of
    the fp64 sum: |got - want| <= K 2^-24 sum|q x| s + a rounding of the result."""
    rng = np.random.default_rng(8)
    M, K, N = 3, 1024, 96
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = rng.uniform(2e-4, 2e-3, N).astype(np.float32)
    x = O.f32_to_f16_bits(rng.standard_normal((M, K)).astype(np.float32))
    out = np.zeros((M, N), np.float32)
    O.lib().orc_gemv_i8w(O.ORC_F16, O._p(q), O._p(s), O._p(x), M, K, N, O._p(out))
    xf = O.f16_bits_to_f32(x).astype(np.float64)
    prod = xf @ q.T.astype(np.float64)
    want = prod * s.astype(np.float64)
    bound = (K * 2.0 ** -24 * (np.abs(xf) @ np.abs(q.T.astype(np.float64))) + 2.0 ** -24 * np.abs(prod)) * s + \
        2.0 ** -24 * np.abs(want)
    assert np.all(np.abs(out - want) <= bound)
    # the scales applied one column off miss it
    assert not np.all(np.abs(out - prod * np.roll(s, 1).astype(np.float64)) <= bound)


def test_rtn_int4_known_answers():
    """orc_rtn_int4_g64 (src/loader/rtn.h) on hand-made groups: amax 7.5 gives the scale 1.0
    exactly, so w / s = w and the ties go to the even integer (0.5 -> 0, 1.5 -> 2, 2.5 -> 2,
    -0.5 -> 0, -1.5 -> -2); +-7.5 clamp to nibbles 15 and 0; amax 1.0 gives the scale
    f16(2/15) = 0x3044; an all-zero group has scale 0 and every nibble 8."""
    K, N = 128, 1
    w = np.zeros(K, np.float32)
    vals = [0.5, 1.5, 2.5, -0.5, -1.5, 7.5, -7.5, 3.0]
    want_q = [8, 10, 10, 8, 6, 15, 0, 11]
    w[:8] = vals
    w[64] = 1.0  # group 1: amax 1.0
    wb = O.f32_to_bf16_bits(w).reshape(N, K)
    q = np.zeros((K // 8, N), np.uint32)
    s = np.zeros((K // 64, N), np.uint16)
    O.lib().orc_rtn_int4_g64(O._p(wb), K, N, O._p(q), O._p(s))
    assert s[0, 0] == 0x3C00 and s[1, 0] == 0x3044
    nib = [(int(q[0, 0]) >> (4 * j)) & 0xF for j in range(8)]
    assert nib == want_q
    assert np.all(q[1:8, 0] == 0x88888888)  # the rest of group 0 is zero: nibble 8
    # group 1: 1.0 / f32(0x3044) = 7.5018... -> 8 + 8 = 16 -> clamped to 15; zeros -> 8
    assert (int(q[8, 0]) & 0xF) == 15 and (int(q[8, 0]) >> 4) == 0x8888888
    zero = np.zeros((1, 64), np.uint16)
    qz = np.zeros((8, 1), np.uint32); sz = np.ones((1, 1), np.uint16)
    O.lib().orc_rtn_int4_g64(O._p(zero), 64, 1, O._p(qz), O._p(sz))
    assert sz[0, 0] == 0 and np.all(qz == 0x88888888)
